"""The rocprofv3 summary tool on small synthetic CSVs: stage attribution of a block's
dispatch sequence, copy calibration of the traffic counters, and the record bench.py
reads back."""
import csv
import json
import re
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "ernie-image-ncnn-vulkan_amd" / "ernie_amd"))
import rocprof_summary as R  # noqa: E402

COPY = "ehip::(anonymous namespace)::convert_kernel(void const*, int, void*, int, unsigned long)"
BLOCK = [
    "_ZN4ehip12_GLOBAL__N_123rmsnorm_pair_k32_kernelIfDF16_Li8EEEvPKT_PKfS6_S6_ifPT0_i",
    "_ZN4ehip8pingpong6kernelIDF16_DF16_Li5EEEvNS0_6ParamsE",
    "_ZN4ehip8pingpong19split_reduce_kernelIDF16_Li0EEEvNS0_6ParamsE",
    "_ZN4ehip12_GLOBAL__N_123qk_rope_permuted_kernelIDF16_EEvPT_iiiillPKfS5_S5_S5_f",
    "_ZN4ehip3sdl6kernelIDF16_Li0EEEvNS0_6ParamsE",
    "_ZN4ehip3sdl14combine_kernelIDF16_EEvNS0_6ParamsEi",
    "_ZN4ehip8pingpong6kernelIDF16_fLi1EEEvNS0_6ParamsE",
    "void ehip::pingpong::split_reduce_kernel<float, 1>(ehip::pingpong::Params)",
    "_ZN4ehip12_GLOBAL__N_123rmsnorm_pair_k32_kernelIfDF16_Li8EEEvPKT_PKfS6_S6_ifPT0_i",
    "_ZN4ehip8pingpong6kernelIDF16_DF16_Li2EEEvNS0_6ParamsE",
    "_ZN4ehip8pingpong19split_reduce_kernelIDF16_Li2EEEvNS0_6ParamsE",
    "_ZN4ehip8pingpong6kernelIDF16_fLi1EEEvNS0_6ParamsE",
    "void ehip::pingpong::split_reduce_kernel<float, 1>(ehip::pingpong::Params)",
]
STAGES = ["rmsnorm_modulate", "gemm_qkv", "gemm_qkv", "gemm_qkv", "sdpa", "sdpa", "gemm_out", "gemm_out",
          "rmsnorm_modulate", "gemm_up_gate", "gemm_up_gate", "gemm_down", "gemm_down"]


def test_stage_attribution_of_a_block():
    prev, got, mains = None, [], 0
    for name in BLOCK * 2:
        st, main = R.stage_of(name, prev)
        got.append(st)
        mains += main
        prev = st
    assert got == STAGES * 2
    assert mains == 2 * 7  # two norms and five stage launches per block
    # A head GEMM's reduction after the last block is no block stage.
    assert R.stage_of("void ehip::pingpong::split_reduce_kernel<float, 0>(ehip::pingpong::Params)", "gemm_down") == \
        (None, False)


# The same block with the launches of the current kernels: GEMM kernels carry the
# heavy-tile flag, reductions their vector width, and the up/gate GEMM (heavy last row
# of tiles) has no reduction after it.
BLOCK_HEAVY = [
    "_ZN4ehip12_GLOBAL__N_123rmsnorm_pair_k32_kernelIfDF16_Li8EEEvPKT_PKfS6_S6_ifPT0_i",
    "_ZN4ehip8pingpong6kernelIDF16_DF16_Li5ELb0EEEvNS0_6ParamsE",
    "_ZN4ehip8pingpong19split_reduce_kernelIDF16_Li0ELi4EEEvNS0_6ParamsE",
    "_ZN4ehip12_GLOBAL__N_123qk_rope_permuted_kernelIDF16_EEvPT_iiiillPKfS5_S5_S5_f",
    "_ZN4ehip3sdl6kernelIDF16_Li0EEEvNS0_6ParamsE",
    "_ZN4ehip3sdl14combine_kernelIDF16_EEvNS0_6ParamsEi",
    "_ZN4ehip8pingpong6kernelIDF16_fLi1ELb0EEEvNS0_6ParamsE",
    "void ehip::pingpong::split_reduce_kernel<float, 1, 4>(ehip::pingpong::Params)",
    "_ZN4ehip12_GLOBAL__N_123rmsnorm_pair_k32_kernelIfDF16_Li8EEEvPKT_PKfS6_S6_ifPT0_i",
    "_ZN4ehip8pingpong6kernelIDF16_DF16_Li2ELb1EEEvNS0_6ParamsE",
    "_ZN4ehip8pingpong6kernelIDF16_fLi1ELb0EEEvNS0_6ParamsE",
    "void ehip::pingpong::split_reduce_kernel<float, 1, 4>(ehip::pingpong::Params)",
]
STAGES_HEAVY = ["rmsnorm_modulate", "gemm_qkv", "gemm_qkv", "gemm_qkv", "sdpa", "sdpa", "gemm_out", "gemm_out",
                "rmsnorm_modulate", "gemm_up_gate", "gemm_down", "gemm_down"]


def test_stage_attribution_of_the_current_kernel_names():
    prev, got = None, []
    for name in BLOCK_HEAVY * 2:
        st, _ = R.stage_of(name, prev)
        got.append(st)
        prev = st
    assert got == STAGES_HEAVY * 2


def write_counters(path, counter, values):
    path.mkdir(parents=True)
    cols = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path / "bench_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for i, (name, v) in enumerate(values):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": v,
                        "Start_Timestamp": 1000 * i, "End_Timestamp": 1000 * i + 500})


def test_traffic_record_scales_by_the_copy_calibration(tmp_path, capsys):
    # Copies of 1 MiB read FETCH 512 KiB (x2) and WRITE 1024 KiB (x1).
    fetch = [(COPY, 512.0)] * 3 + [(n, 100.0 * (i + 1)) for i, n in enumerate(BLOCK)]
    write = [(COPY, 1024.0)] * 3 + [(n, 10.0) for n in BLOCK]
    write_counters(tmp_path / "f", "FETCH_SIZE", fetch)
    write_counters(tmp_path / "w", "WRITE_SIZE", write)
    R.main(["traffic", str(tmp_path / "f"), str(tmp_path / "w"), "--copy-mib", "1", "--sources-sha256", "abc",
            "--command", "cmd"])
    out = capsys.readouterr().out
    rec = json.loads(re.search(r"```json traffic\n(.*?)\n```", out, re.S).group(1))
    assert rec["kernel_sources_sha256"] == "abc"
    kib = 1024
    expect_qkv = (200 + 300 + 400) * kib * 2 + 3 * 10 * kib
    assert rec["bytes_per_launch"]["gemm_qkv"] == expect_qkv
    assert rec["bytes_per_launch"]["rmsnorm_modulate"] == ((100 + 900) * kib * 2 + 2 * 10 * kib) // 2
    assert rec["bytes_per_launch"]["gemm_down"] == (1200 + 1300) * kib * 2 + 2 * 10 * kib


def test_traffic_refuses_runs_without_the_calibration(tmp_path):
    write_counters(tmp_path / "f", "FETCH_SIZE", [(n, 1.0) for n in BLOCK])
    write_counters(tmp_path / "w", "WRITE_SIZE", [(n, 1.0) for n in BLOCK])
    with pytest.raises(SystemExit):
        R.main(["traffic", str(tmp_path / "f"), str(tmp_path / "w"), "--sources-sha256", "abc"])
