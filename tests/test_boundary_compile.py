"""The documented reference-side binding compiles against the reference and
behaves as the reference's backend contract says (CPU only).

INTEGRATION.md section 1 holds `hillserve::GpuBackend : FpgaScoreBackend`,
the class a reference maintainer adds to route `FullGqaRuntimePolicy`'s device
scorer to this library.  This test cuts that block out of INTEGRATION.md (so
the document cannot drift from what is compiled), compiles it with the
reference's own `smartssd/adapter.hpp` and `smartssd/stream_layout.hpp`
(read in place under /root/reference, nothing copied) plus a driver written
here, links `libhillserve_amd.so`, and runs the driver without a GPU:

* through a `FpgaScoreBackend` pointer, every shape the reference's
  `validate_raw_gqa_shape` (smartssd/adapter.hpp:97-104) refuses is refused
  with the same exception type and text, under both ABIs;
* the per-query-head partial layout is refused; the methods the GPU backend
  does not serve keep the base class's throwing defaults;
* the chunk planner behind the streamed method equals the reference's
  header-only `plan_raw_gqa_stream` (smartssd/stream_layout.hpp:18-51) on
  300 random region lists: the same reads, offsets, sizes and destinations,
  or the same exception type when the layout is refused, also when called
  through the backend's streamed method.

Skipped where /root/reference is absent (the GPU box); nothing in the product
links or reads the reference."""
import os
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

DRIVER = r'''
#include <iostream>
#include <random>
#include <string>
#include <utility>

#include "smartssd/adapter.hpp"
#include "smartssd/stream_layout.hpp"
#include "hs_gqa.hpp"

namespace hillserve {
std::unique_ptr<FpgaScoreBackend> make_gpu_score_backend(const HardwareContract& c);
}

namespace {
int failures = 0, checks = 0;
void check(bool ok, const std::string& what) {
    ++checks;
    if (!ok) {
        ++failures;
        std::cerr << "FAILED: " << what << std::endl;
    }
}
template <class F>
std::pair<std::string, std::string> thrown(F f) {
    try {
        f();
    } catch (const std::length_error& e) {
        return {"length_error", e.what()};
    } catch (const std::invalid_argument& e) {
        return {"invalid_argument", e.what()};
    } catch (const std::runtime_error& e) {
        return {"runtime_error", e.what()};
    } catch (const std::exception& e) {
        return {"exception", e.what()};
    }
    return {"none", ""};
}
}  // namespace

int main() {
    using namespace hillserve;
    for (const std::string abi : {"HS_FULL_GQA_PIPELINE_F16_V3", "HS_FULL_GQA_F16_V2"}) {
        HardwareContract c;
        c.abi = abi;
        std::unique_ptr<FpgaScoreBackend> b = make_gpu_score_backend(c);
        const std::vector<std::uint16_t> q(32 * 128), k;
        const std::size_t shapes[][4] = {{32, 8, 0, 128},  {32, 8, 100, 128}, {32, 8, 32832, 128},
                                         {16, 8, 64, 128}, {32, 4, 64, 128},  {32, 8, 64, 64},
                                         {32, 8, 32, 128}, {32, 8, 65, 128}};
        for (const auto& s : shapes) {
            const auto want = thrown([&] { validate_raw_gqa_shape(abi, s[0], s[1], s[2], s[3]); });
            if (want.first == "none") continue;  // accepted shapes need a GPU
            const auto got = thrown([&] { b->score_raw_gqa(q, k, s[0], s[1], s[2], s[3]); });
            check(got == want, abi + " shape rejection: " + got.first + " '" + got.second +
                                   "' against the reference's '" + want.second + "'");
        }
        check(thrown([&] { b->score(q, k, 32, 64, 128); }).first == "invalid_argument",
              "partial layout refused");
        const ScoreFileRegion region{3, 0, 64 * 2048, false};
        check(thrown([&] { b->score_file_raw_gqa(q, region, 32, 8, 64, 128); }) ==
                  std::make_pair(std::string("invalid_argument"),
                                 std::string("full raw GQA file ABI unavailable in this backend")),
              "base default of score_file_raw_gqa");
        check(thrown([&] { b->score_resident_file(q, 32, 8, 128); }).first == "runtime_error",
              "base default of score_resident_file");
        check(thrown([&] { b->score_file(q, region, 32, 64, 128); }).first == "runtime_error",
              "base default of score_file");
    }

    // the planner behind the streamed method against the reference's planner
    std::mt19937_64 gen(2024);
    const std::size_t block = 64 * 2048;
    HardwareContract c;
    c.abi = "HS_FULL_GQA_PIPELINE_F16_V3";
    std::unique_ptr<FpgaScoreBackend> b = make_gpu_score_backend(c);
    int planned = 0, refused = 0;
    for (int trial = 0; trial < 300; ++trial) {
        const int count = 1 + int(gen() % 6);
        std::vector<ScoreFileRegion> regions;
        std::vector<gpu::ScoreFileRegion> ours;
        std::uint64_t next[3] = {0, 0, 0};
        for (int i = 0; i < count; ++i) {
            const int fd = 3 + int(gen() % 3);
            std::uint64_t blocks = 1 + gen() % 96, offset = next[fd - 3];
            if (gen() % 3 == 0) offset += 4096 * (gen() % 64);  // a gap in the file
            if (gen() % 4 == 0) offset = (gen() % 512) * 4096;   // anywhere, even backwards
            std::uint64_t bytes = blocks * block;
            int bad = int(gen() % 40);
            if (bad == 0) offset += 8;        // unaligned offset
            if (bad == 1) bytes -= 4096;      // partial block
            if (bad == 2) bytes = 0;          // empty region
            next[fd - 3] = offset + bytes;
            regions.push_back({bad == 3 ? -1 : fd, offset, bytes, false});
            ours.push_back({regions.back().fd, offset, bytes, false});
        }
        std::size_t chunk = 64 * (1 + gen() % 512);
        const int bad_chunk = int(gen() % 30);
        if (bad_chunk == 0) chunk = 0;
        if (bad_chunk == 1) chunk += 1;
        if (bad_chunk == 2) chunk = 32768 + 64;
        std::vector<DirectChunkPlan> want;
        std::vector<gpu::DirectChunkPlan> got;
        const auto e_want = thrown([&] { want = plan_raw_gqa_stream(regions, chunk); });
        const auto e_got = thrown([&] { got = gpu::plan_raw_gqa_stream(ours, chunk); });
        check(e_want.first == e_got.first,
              "trial " + std::to_string(trial) + ": planner outcome " + e_got.first +
                  " against the reference's " + e_want.first);
        if (e_want.first != "none") {
            ++refused;
            const std::vector<std::uint16_t> q(32 * 128);
            const auto via = thrown([&] {
                b->score_file_regions_raw_gqa_stream(q, regions, 32, 8, 128, chunk,
                                                     [](const FileScoreChunk&) {});
            });
            check(via.first == e_want.first, "trial " + std::to_string(trial) +
                                                 ": the streamed method refuses as the planner");
            continue;
        }
        ++planned;
        bool same = want.size() == got.size();
        for (std::size_t i = 0; same && i < want.size(); ++i) {
            same = want[i].token_offset == got[i].token_offset && want[i].tokens == got[i].tokens &&
                   want[i].reads.size() == got[i].reads.size();
            for (std::size_t j = 0; same && j < want[i].reads.size(); ++j) {
                const auto& x = want[i].reads[j];
                const auto& y = got[i].reads[j];
                same = x.fd == y.fd && x.offset == y.offset && x.bytes == y.bytes &&
                       x.destination_offset == y.destination_offset;
            }
        }
        check(same, "trial " + std::to_string(trial) + ": plans differ from the reference's");
    }
    std::cout << "{\"checks\":" << checks << ",\"failures\":" << failures
              << ",\"planned\":" << planned << ",\"refused\":" << refused << "}" << std::endl;
    return failures ? 1 : 0;
}
'''


def binding_block() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    m = re.search(r"```cpp\n(// smartssd/gpu_backend\.cpp.*?)```", text, re.S)
    assert m, "INTEGRATION.md lost its GpuBackend block"
    return m.group(1)


@pytest.mark.skipif(not (REF / "smartssd" / "adapter.hpp").exists(),
                    reason="the reference tree is not here (it never travels to the GPU box)")
def test_documented_binding_compiles_and_keeps_the_contract(tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("CPU-only contract check (a GPU is visible)")
    lib_dir = ROOT / "hillserve_amd"
    assert (lib_dir / "libhillserve_amd.so").exists(), "run python -m hillserve_amd.build"
    backend = tmp_path / "gpu_backend.cpp"
    backend.write_text(binding_block())
    driver = tmp_path / "driver.cpp"
    driver.write_text(DRIVER)
    exe = tmp_path / "binding"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", f"-I{REF}", f"-I{ROOT / 'include'}",
                    f"-I{ROCM / 'include'}", "-D__HIP_PLATFORM_AMD__", str(backend), str(driver),
                    str(REF / "smartssd" / "adapter.cpp"), f"-L{lib_dir}", "-lhillserve_amd",
                    f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{lib_dir}:{ROCM / 'lib'}",
                    "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert '"failures":0' in proc.stdout and '"planned":' in proc.stdout, proc.stdout
