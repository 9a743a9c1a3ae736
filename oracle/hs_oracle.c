/*
 * hs_oracle.c — CPU restatement of the HillServe sparse-KV hot path.
 * TEST INFRASTRUCTURE ONLY (see hs_oracle.h for who may load it and for the
 * checks that pin each function).  Compiled with -ffp-contract=off.
 */
#include "hs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- binary16 <-> binary32 (policy/host_policy.cpp:9-28) ---------------- */

float hso_half_value(uint16_t h)
{
    const uint32_t exponent = (h >> 10) & 31u;
    const uint32_t fraction = h & 1023u;
    if (exponent == 0) {
        /* zero or subnormal: fraction * 2^-24 is exact in FP32 */
        const float magnitude = (float)fraction * 0x1p-24f;
        return (h & 0x8000u) ? -magnitude : magnitude;
    }
    uint32_t bits = (uint32_t)(h & 0x8000u) << 16;
    if (exponent == 31)
        bits |= 0x7f800000u | (fraction << 13);
    else
        bits |= ((exponent + 112u) << 23) | (fraction << 13);
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

uint16_t hso_half_bits(float f)
{
    uint32_t v;
    memcpy(&v, &f, sizeof v);
    const uint32_t sign = (v >> 16) & 0x8000u;
    const uint32_t biased = (v >> 23) & 255u;
    uint32_t mantissa = v & 0x7fffffu;
    if (biased == 255) /* inf keeps its sign; NaN becomes sign|0x7e00 */
        return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u : 0u));
    const int e = (int)biased - 112; /* rebias 127 -> 15 */
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    uint32_t kept, dropped, half;
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        mantissa |= 0x800000u;
        const unsigned shift = (unsigned)(14 - e);
        kept = mantissa >> shift;
        dropped = mantissa & ((1u << shift) - 1u);
        half = 1u << (shift - 1u);
    } else {
        kept = ((uint32_t)e << 10) | (mantissa >> 13);
        dropped = mantissa & 0x1fffu;
        half = 0x1000u;
    }
    const uint32_t up = dropped > half || (dropped == half && (kept & 1u));
    return (uint16_t)(sign | (kept + up));
}

/* policy/half_order.hpp:7-10 */
uint16_t hso_order_key(uint16_t bits)
{
    if ((bits & 0x7fffu) == 0)
        bits = 0;
    return (bits & 0x8000u) ? (uint16_t)~bits : (uint16_t)(bits ^ 0x8000u);
}

/* ---- raw scores (policy/full_gqa_cpu.cpp:23-37, kernel.cpp:152-198) ----- */

int hso_score(const uint16_t *q, const uint16_t *k, size_t stride_words,
              size_t n, uint16_t *out, size_t out_stride)
{
    if (!q || !k || !out || n == 0 || out_stride < n ||
        (stride_words != 1024 && stride_words != 2048))
        return HSO_ERR_SHAPE;
    float qf[32 * 128];
    for (size_t i = 0; i < 32 * 128; ++i)
        qf[i] = hso_half_value(q[i]);
    for (size_t t = 0; t < n; ++t) {
        const uint16_t *row = k + t * stride_words;
        for (size_t h = 0; h < 32; ++h) {
            const uint16_t *key = row + (h / 4) * 128;
            const float *qh = qf + h * 128;
            float sum = 0.0f;
            for (size_t c = 0; c < 128; ++c) {
                const float product = qh[c] * hso_half_value(key[c]);
                sum = sum + product;
            }
            out[h * out_stride + t] = hso_half_bits(sum);
        }
    }
    return HSO_OK;
}

/* ---- scaling (policy/full_gqa_runtime.cpp:571) -------------------------- */

uint16_t hso_scale_one(uint16_t raw)
{
    const float root = sqrtf(128.0f);
    return hso_half_bits(hso_half_value(raw) / root);
}

void hso_scale(const uint16_t *raw, uint16_t *scaled, size_t count)
{
    for (size_t i = 0; i < count; ++i)
        scaled[i] = hso_scale_one(raw[i]);
}

/* ---- selector (policy/gqa_policy.cpp:47-70) ----------------------------- */

static int is_finite_f(float x) { return isfinite(x) != 0; }

static int selector_k(const uint16_t *s, size_t heads, size_t stride, size_t n,
                      float alpha, float ratio, int fp32_counts,
                      uint32_t *counts, size_t *k_out)
{
    if (!s || heads == 0 || heads > 128 || n == 0 || n > stride)
        return HSO_ERR_SHAPE;
    if (!is_finite_f(alpha) || alpha < 0 || !is_finite_f(ratio) || ratio <= 0 ||
        ratio > 1)
        return HSO_ERR_SHAPE;
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        const float x = hso_half_value(s[i]);
        if (!is_finite_f(x))
            return HSO_ERR_NONFINITE;
        maximum = maximum > x ? maximum : x;
    }
    const float threshold = hso_half_value(hso_half_bits(maximum - alpha));
    if (!is_finite_f(threshold))
        return HSO_ERR_THRESHOLD;
    float total = 0.0f;
    for (size_t h = 0; h < heads; ++h) {
        uint64_t count = 0;
        for (size_t i = 0; i < n; ++i) {
            const float x = hso_half_value(s[h * stride + i]);
            if (!is_finite_f(x))
                return HSO_ERR_NONFINITE;
            count += x >= threshold;
        }
        if (counts)
            counts[h] = (uint32_t)count;
        const float rounded = fp32_counts
                                  ? (float)count
                                  : hso_half_value(hso_half_bits((float)count));
        if (!is_finite_f(rounded))
            return HSO_ERR_COUNT;
        total += rounded;
    }
    const float mean = fp32_counts
                           ? total / (float)heads
                           : hso_half_value(hso_half_bits(total / (float)heads));
    if (!is_finite_f(mean))
        return HSO_ERR_MEAN;
    size_t k = (size_t)mean;
    const size_t cap = (size_t)floor((double)n * (double)ratio);
    if (cap < k)
        k = cap;
    if (n < k)
        k = n;
    *k_out = k;
    return HSO_OK;
}

int hso_select_k(const uint16_t *scaled, size_t heads, size_t stride, size_t n,
                 float alpha, float ratio, int fp32_counts, size_t *k_out)
{
    return selector_k(scaled, heads, stride, n, alpha, ratio, fp32_counts, NULL,
                      k_out);
}

int hso_select(const uint16_t *scaled, size_t heads, size_t stride, size_t n,
               float alpha, float ratio, int fp32_counts, uint32_t *ids,
               size_t ids_stride, uint32_t *counts, size_t *k_out,
               size_t *tied_out)
{
    size_t k = 0;
    const int rc = selector_k(scaled, heads, stride, n, alpha, ratio,
                              fp32_counts, counts, &k);
    if (rc != HSO_OK)
        return rc;
    if (ids_stride < k)
        return HSO_ERR_SHAPE;
    /* Stable counting sort on the 16-bit order key, descending, visiting ids
     * in ascending order: position p holds the p-th element of the order
     * (key desc, id asc).  Positions 0..k are needed (k for the tie check). */
    uint32_t *start = (uint32_t *)malloc(sizeof(uint32_t) * 65536);
    uint32_t *first = (uint32_t *)malloc(sizeof(uint32_t) * (k + 1));
    if (!start || !first) {
        free(start);
        free(first);
        return HSO_ERR_SHAPE;
    }
    size_t tied = 0;
    for (size_t h = 0; h < heads; ++h) {
        const uint16_t *row = scaled + h * stride;
        memset(start, 0, sizeof(uint32_t) * 65536);
        for (size_t i = 0; i < n; ++i)
            start[hso_order_key(row[i])]++;
        uint32_t running = 0;
        for (int key = 65535; key >= 0; --key) {
            const uint32_t c = start[key];
            start[key] = running;
            running += c;
        }
        for (size_t i = 0; i < n; ++i) {
            const uint32_t p = start[hso_order_key(row[i])]++;
            if (p <= k)
                first[p] = (uint32_t)i;
        }
        if (k && k < n && row[first[k - 1]] == row[first[k]])
            ++tied;
        if (ids)
            memcpy(ids + h * ids_stride, first, sizeof(uint32_t) * k);
    }
    free(start);
    free(first);
    *k_out = k;
    if (tied_out)
        *tied_out = tied;
    return HSO_OK;
}

/* ---- history cover (policy/full_gqa_runtime.cpp:299-344) ---------------- */

int hso_history_cover(const uint16_t *raw, size_t heads, size_t stride,
                      size_t position, float alpha, float ratio, int fp32_counts,
                      uint32_t *ids, size_t ids_stride, size_t *bound_out,
                      uint32_t *physical, size_t *physical_n)
{
    /* :309-311 cap over position + 1 columns; position < capacity */
    if (!raw || heads == 0 || heads > 128 || position == 0 || position >= stride)
        return HSO_ERR_SHAPE;
    size_t cap = (size_t)floor((double)(position + 1) * (double)ratio);
    if (position < cap)
        cap = position;
    if (cap == 0)
        return HSO_ERR_SHAPE;
    /* :312 scaling */
    uint16_t *scaled = (uint16_t *)malloc(sizeof(uint16_t) * heads * stride);
    if (!scaled)
        return HSO_ERR_SHAPE;
    for (size_t i = 0; i < heads * stride; ++i)
        scaled[i] = hso_scale_one(raw[i]);
    /* :313-314 head-0 maximum as std::max(maximum, x): NaN never replaces it */
    float maximum = -INFINITY;
    for (size_t t = 0; t < position; ++t) {
        const float x = hso_half_value(scaled[t]);
        if (maximum < x)
            maximum = x;
    }
    /* :315-316 threshold */
    const float threshold = hso_half_value(hso_half_bits(maximum - alpha));
    int rc = HSO_OK;
    if (!is_finite_f(threshold))
        rc = HSO_ERR_THRESHOLD;
    /* :317-324 counts with one possible current token each */
    float count_sum = 0.0f;
    for (size_t h = 0; rc == HSO_OK && h < heads; ++h) {
        uint64_t count = 1;
        for (size_t t = 0; t < position; ++t)
            count += hso_half_value(scaled[h * stride + t]) >= threshold;
        const float rounded = fp32_counts ? (float)count
                                          : hso_half_value(hso_half_bits((float)count));
        if (!is_finite_f(rounded))
            rc = HSO_ERR_COUNT;
        count_sum += rounded;
    }
    size_t bound = 0;
    if (rc == HSO_OK) {
        /* :325-327 mean bound, :328 bound */
        const float mean = fp32_counts
                               ? count_sum / (float)heads
                               : hso_half_value(hso_half_bits(count_sum / (float)heads));
        if (!is_finite_f(mean) || !(mean >= 1.0f))
            rc = HSO_ERR_MEAN;
        else
            bound = (size_t)mean < cap ? (size_t)mean : cap;
    }
    if (rc == HSO_OK && ids && ids_stride < bound)
        rc = HSO_ERR_SHAPE;
    if (rc != HSO_OK) {
        free(scaled);
        return rc;
    }
    /* :329-337 per head, the first `bound` of (key desc, id asc): stable
     * counting sort on the order key, ids visited ascending */
    uint32_t *start = (uint32_t *)malloc(sizeof(uint32_t) * 65536);
    unsigned char *used = (unsigned char *)calloc(position, 1);
    if (!start || !used) {
        free(start);
        free(used);
        free(scaled);
        return HSO_ERR_SHAPE;
    }
    for (size_t h = 0; h < heads; ++h) {
        const uint16_t *row = scaled + h * stride;
        memset(start, 0, sizeof(uint32_t) * 65536);
        for (size_t t = 0; t < position; ++t)
            start[hso_order_key(row[t])]++;
        uint32_t running = 0;
        for (int key = 65535; key >= 0; --key) {
            const uint32_t c = start[key];
            start[key] = running;
            running += c;
        }
        for (size_t t = 0; t < position; ++t) {
            const uint32_t p = start[hso_order_key(row[t])]++;
            if (p < bound) {
                if (ids)
                    ids[h * ids_stride + p] = (uint32_t)t;
                used[t] = 1;
            }
        }
    }
    /* :338-340 the sorted union */
    size_t np = 0;
    for (size_t t = 0; t < position; ++t)
        if (used[t]) {
            if (physical)
                physical[np] = (uint32_t)t;
            ++np;
        }
    if (physical_n)
        *physical_n = np;
    *bound_out = bound;
    free(start);
    free(used);
    free(scaled);
    return HSO_OK;
}

/* ---- cold tier format (storage/segmented_store.cpp:18-38, file_store.cpp:12) */

uint64_t hso_fnv1a64(const uint8_t *p, size_t n)
{
    uint64_t h = 14695981039346656037ULL;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 1099511628211ULL;
    }
    return h;
}

static void put_u64(uint8_t *dst, uint64_t v)
{
    for (int b = 0; b < 8; ++b)
        dst[b] = (uint8_t)(v >> (8 * b));
}

uint64_t hso_kv_store_extent(size_t layers, size_t positions)
{
    return (4096u + (uint64_t)layers * positions * 4128u + 4095u) / 4096u * 4096u;
}

void hso_kv_store_header(uint8_t *page, uint64_t request, size_t layers, size_t positions)
{
    memset(page, 0, 4096);
    put_u64(page + 0, 0x48534b5653454731ULL);
    put_u64(page + 8, 1);
    put_u64(page + 16, request);
    put_u64(page + 24, layers);
    put_u64(page + 32, positions);
    put_u64(page + 40, 4096);
    put_u64(page + 48, 4128);
    put_u64(page + 56, hso_kv_store_extent(layers, positions));
}

void hso_kv_record(uint8_t *out, const uint8_t *row, uint64_t position, uint64_t request,
                   uint32_t layer)
{
    put_u64(out + 0, hso_fnv1a64(row, 4096));
    put_u64(out + 8, position);
    put_u64(out + 16, request);
    for (int b = 0; b < 4; ++b) {
        out[24 + b] = (uint8_t)(layer >> (8 * b));
        out[28 + b] = (uint8_t)(1u >> (8 * b));
    }
    memcpy(out + 32, row, 4096);
}

/* ---- union and pack (runtime/gqa_pack.hpp:12-58) ------------------------ */

int hso_physical_union(const uint32_t *ids, const size_t *lens,
                       size_t ids_stride, size_t visible, uint32_t *out,
                       size_t *out_n)
{
    if (!visible || visible > 66048)
        return HSO_ERR_SHAPE;
    uint32_t *seen = (uint32_t *)calloc(visible, sizeof(uint32_t));
    if (!seen)
        return HSO_ERR_SHAPE;
    for (size_t h = 0; h < 32; ++h) {
        const uint32_t bit = 1u << h;
        for (size_t j = 0; j < lens[h]; ++j) {
            const uint32_t id = ids[h * ids_stride + j];
            if (id >= visible || (seen[id] & bit)) {
                free(seen);
                return HSO_ERR_DUPLICATE;
            }
            seen[id] |= bit;
        }
    }
    size_t m = 0;
    for (size_t i = 0; i < visible; ++i)
        if (seen[i])
            out[m++] = (uint32_t)i;
    free(seen);
    *out_n = m;
    return HSO_OK;
}

int hso_pack(const uint32_t *ids, const size_t *lens, size_t ids_stride,
             const uint64_t *positions, size_t nq, const uint32_t *physical,
             size_t np, const uint8_t *payload, size_t count, uint16_t *k_out,
             uint16_t *v_out, float *mask)
{
    if (nq == 0 || nq > 256 || positions[nq - 1] >= 66048 || count == 0 ||
        count > 66048)
        return HSO_ERR_SHAPE;
    const size_t extent = (size_t)positions[nq - 1] + 1;
    int32_t *offset = (int32_t *)malloc(sizeof(int32_t) * extent);
    if (!offset)
        return HSO_ERR_SHAPE;
    for (size_t i = 0; i < extent; ++i)
        offset[i] = -1;
    for (size_t i = 0; i < np; ++i) {
        const uint32_t id = physical[i];
        if (id >= extent || offset[id] != -1) {
            free(offset);
            return HSO_ERR_DUPLICATE;
        }
        offset[id] = (int32_t)i;
    }
    const size_t qpad = (nq + 63) / 64 * 64;
    memset(k_out, 0, sizeof(uint16_t) * count * 4096);
    memset(v_out, 0, sizeof(uint16_t) * count * 4096);
    for (size_t i = 0; i < count * qpad * 32; ++i)
        mask[i] = -INFINITY;
    for (size_t h = 0; h < 32; ++h) {
        if (lens[h] == 0 || lens[h] > count) {
            free(offset);
            return HSO_ERR_SHAPE;
        }
        const size_t kv = h / 4;
        for (size_t s = 0; s < lens[h]; ++s) {
            const uint32_t id = ids[h * ids_stride + s];
            if (id >= extent || offset[id] < 0) {
                free(offset);
                return HSO_ERR_MISSING;
            }
            const uint8_t *src = payload + (size_t)offset[id] * 4096;
            memcpy(k_out + s * 4096 + h * 128, src + kv * 256, 256);
            for (size_t d = 0; d < 128; ++d)
                memcpy(v_out + (h * 128 + d) * count + s,
                       src + 2048 + (kv * 128 + d) * 2, 2);
            for (size_t qi = 0; qi < nq; ++qi)
                if (id <= positions[qi])
                    mask[(h * qpad + qi) * count + s] = 0.0f;
        }
    }
    free(offset);
    return HSO_OK;
}

/* runtime/gqa_prefetch_cuda.cu:12-22 */
void hso_gather_rows(const uint16_t *prefetched, const uint16_t *misses,
                     const int32_t *map, size_t count, uint16_t *k_out,
                     uint16_t *v_out)
{
    for (size_t s = 0; s < count; ++s)
        for (size_t h = 0; h < 32; ++h) {
            const int32_t row = map[h * count + s];
            const uint16_t *src = NULL;
            if (row >= 0)
                src = prefetched + (size_t)row * 2048;
            else if (row <= -2)
                src = misses + (size_t)(-2 - (int64_t)row) * 2048;
            for (size_t d = 0; d < 128; ++d) {
                const uint16_t kv_k = src ? src[(h / 4) * 128 + d] : 0;
                const uint16_t kv_v = src ? src[1024 + (h / 4) * 128 + d] : 0;
                k_out[(s * 32 + h) * 128 + d] = kv_k;
                v_out[(h * 128 + d) * count + s] = kv_v;
            }
        }
}

/* ---- FP64 attention over a selection ------------------------------------ */

void hso_attention_f64(const float *q, const uint8_t *pool, size_t row_bytes,
                       const int32_t *rows, const uint32_t *ids,
                       const size_t *lens, size_t ids_stride, double *out)
{
    const double scale = 1.0 / sqrt(128.0);
    for (size_t h = 0; h < 32; ++h) {
        const size_t kv = h / 4, m = lens[h];
        double *o = out + h * 128;
        /* an empty selection: NaN, the fully masked softmax row */
        for (size_t d = 0; d < 128; ++d)
            o[d] = m == 0 ? NAN : 0.0;
        if (m == 0)
            continue;
        double *s = (double *)malloc(sizeof(double) * m);
        double top = -INFINITY;
        for (size_t j = 0; j < m; ++j) {
            const uint32_t id = ids[h * ids_stride + j];
            const size_t r = rows ? (size_t)rows[id] : id;
            const uint16_t *key =
                (const uint16_t *)(pool + r * row_bytes) + kv * 128;
            double dot = 0.0;
            for (size_t c = 0; c < 128; ++c)
                dot += (double)q[h * 128 + c] * (double)hso_half_value(key[c]);
            s[j] = dot * scale;
            top = s[j] > top ? s[j] : top;
        }
        double total = 0.0;
        for (size_t j = 0; j < m; ++j) {
            s[j] = exp(s[j] - top);
            total += s[j];
        }
        for (size_t j = 0; j < m; ++j) {
            const uint32_t id = ids[h * ids_stride + j];
            const size_t r = rows ? (size_t)rows[id] : id;
            const uint16_t *value =
                (const uint16_t *)(pool + r * row_bytes + 2048) + kv * 128;
            const double p = s[j] / total;
            for (size_t d = 0; d < 128; ++d)
                o[d] += p * (double)hso_half_value(value[d]);
        }
        free(s);
    }
}

/* ---- rehearsal query (config 4), FP64 ----------------------------------- */

static double bf16_value(uint16_t b)
{
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return (double)f;
}

void hso_rehearsal_f64(const uint16_t *hidden_bf16, const uint16_t *wq_bf16,
                       double eps, double theta, uint64_t pos, double *out)
{
    double x[4096];
    double sq = 0.0;
    for (size_t i = 0; i < 4096; ++i) {
        x[i] = bf16_value(hidden_bf16[i]);
        sq += x[i] * x[i];
    }
    const double inv = 1.0 / sqrt(sq / 4096.0 + eps);
    for (size_t i = 0; i < 4096; ++i)
        x[i] *= inv;
    for (size_t o = 0; o < 4096; ++o) {
        double acc = 0.0;
        const uint16_t *w = wq_bf16 + o * 4096;
        for (size_t i = 0; i < 4096; ++i)
            acc += bf16_value(w[i]) * x[i];
        out[o] = acc;
    }
    for (size_t h = 0; h < 32; ++h)
        for (size_t i = 0; i < 64; ++i) {
            const double angle =
                (double)pos * pow(theta, -2.0 * (double)i / 128.0);
            const double c = cos(angle), s = sin(angle);
            double *pair = out + h * 128 + 2 * i;
            const double a = pair[0], b = pair[1];
            pair[0] = a * c - b * s;
            pair[1] = a * s + b * c;
        }
}

/* ---- exhaustive FP32 -> F16 check against F16C --------------------------- */

#if defined(__x86_64__) || defined(__i386__)
#include <immintrin.h>
__attribute__((target("f16c"))) static uint16_t f16c_convert(float f)
{
    return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
}
struct sweep {
    uint64_t begin, end;
    long long mismatches;
};
static void *sweep_worker(void *arg)
{
    struct sweep *w = (struct sweep *)arg;
    long long bad = 0;
    for (uint64_t b = w->begin; b < w->end; ++b) {
        const uint32_t bits = (uint32_t)b;
        if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu))
            continue; /* NaN: F16C keeps payload, the reference canonicalizes */
        float f;
        memcpy(&f, &bits, sizeof f);
        bad += hso_half_bits(f) != f16c_convert(f);
    }
    w->mismatches = bad;
    return NULL;
}
long long hso_check_half_bits_f16c(unsigned threads)
{
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("f16c"))
        return -1;
    if (threads == 0 || threads > 64)
        threads = 1;
    pthread_t tid[64];
    struct sweep work[64];
    const uint64_t total = 1ull << 32;
    for (unsigned i = 0; i < threads; ++i) {
        work[i].begin = total * i / threads;
        work[i].end = total * (i + 1) / threads;
        work[i].mismatches = 0;
        pthread_create(&tid[i], NULL, sweep_worker, &work[i]);
    }
    long long bad = 0;
    for (unsigned i = 0; i < threads; ++i) {
        pthread_join(tid[i], NULL);
        bad += work[i].mismatches;
    }
    return bad;
}
#else
long long hso_check_half_bits_f16c(unsigned threads)
{
    (void)threads;
    return -1;
}
#endif

/* ---- fold of hso_half_bits over all FP32 patterns ------------------------ */

struct fold {
    uint64_t *out;
    uint32_t first, last; /* high halves [first, last) */
};
static void *fold_worker(void *arg)
{
    struct fold *w = (struct fold *)arg;
    for (uint32_t hi = w->first; hi < w->last; ++hi) {
        uint64_t acc = 0;
        for (uint32_t lo = 0; lo < 65536; ++lo) {
            const uint32_t bits = (hi << 16) | lo;
            if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu))
                continue;
            float f;
            memcpy(&f, &bits, sizeof f);
            acc += (uint64_t)(hso_half_bits(f) + 1u) * (uint64_t)(lo + 1u);
        }
        w->out[hi] = acc;
    }
    return NULL;
}
void hso_f16_checksums(uint64_t *out, unsigned threads)
{
    if (threads == 0 || threads > 64)
        threads = 1;
    pthread_t tid[64];
    struct fold work[64];
    for (unsigned i = 0; i < threads; ++i) {
        work[i].out = out;
        work[i].first = (uint32_t)(65536ull * i / threads);
        work[i].last = (uint32_t)(65536ull * (i + 1) / threads);
        pthread_create(&tid[i], NULL, fold_worker, &work[i]);
    }
    for (unsigned i = 0; i < threads; ++i)
        pthread_join(tid[i], NULL);
}
