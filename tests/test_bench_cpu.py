"""bench.py's contract pieces that need no GPU: the one-GPU refusal and the
algorithmic bytes and flops its roofline fractions divide by.

The byte counts follow the per-call formula K*N*bits/8 + 4*(#scales) + 4*M*K
+ 4*M*N (+ 4*N bias), #scales = 1 (per tensor), K (per row) or K*N/G (INT4
groups along the flattened [K, N], src/quantization.cpp:113-159), worked out
by hand below for each BASELINE config.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def _run_bench(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          env=env, timeout=120)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = _run_bench(args, env)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no bench line


def test_algorithmic_bytes_and_flops():
    import bench

    c = bench.CONFIGS
    # C1: 1024x1024 INT8 codes, one per-tensor scale, x 128x1024, y 128x1024, bias 1024.
    assert bench.alg_bytes(c["c1"]) == 1024 * 1024 + 4 + 4 * 128 * 1024 + 4 * 128 * 1024 + 4 * 1024 == 2_101_252
    # C2: 4096x4096 nibbles, 131072 group scales, x and y of 4096.
    assert bench.alg_bytes(c["c2"]) == 8_388_608 + 524_288 + 16_384 + 16_384 == 8_945_664
    # C3 gate at M=1: 4096x11008 nibbles, 352256 group scales, x 4096, y 11008.
    assert bench.alg_bytes(c["c3_gate_m1"]) == 22_544_384 + 1_409_024 + 4 * 4096 + 4 * 11008 == 24_013_824
    # C4: 4096x4096 INT8 codes, one scale, x and y of 2048x4096.
    assert bench.alg_bytes(c["c4"]) == 16_777_216 + 4 + 2 * 4 * 2048 * 4096 == 83_886_084
    assert bench.alg_flops(c["c4"]) == 2 * 2048 * 4096 * 4096 == 68_719_476_736
    assert bench.alg_flops(c["c2"]) == 2 * 4096 * 4096


def test_size_sweep_starts_at_c2():
    import bench

    K, N = bench.GEMV_SWEEP[0]
    assert (K, N) == (bench.CONFIGS["c2"]["K"], bench.CONFIGS["c2"]["N"])
    codes = [K * N // 2 for K, N in bench.GEMV_SWEEP]
    assert codes == sorted(codes)
    assert codes[-1] > 256_000_000  # the largest weight alone exceeds the 256 MB Infinity Cache


def test_committed_profiles_count_only_for_the_kernels_they_measured():
    """A kernel-trace or traffic profile names the digest of the kernel
    sources it measured; bench.py reports its figures as this build's only
    when that digest is the current one, else under rocprof_historical."""
    import bench

    cur = bench.csrc_digest()
    assert len(cur) == 16 and cur == bench.csrc_digest()
    prof = {"kernel": "k", "avg_ns_graph_replays": 4000, "summary": "s", "csrc_digest": cur}
    r = bench.rocprof_fields(prof, 8e6, 8000.0, lambda bps: bps / 1e9)
    assert r["kernel_ns_rocprof"] == 4000 and abs(r["frac_kernel_rocprof"] - 0.25) < 1e-9
    stale = dict(prof, csrc_digest="0" * 16)
    r = bench.rocprof_fields(stale, 8e6, 8000.0, lambda bps: bps / 1e9)
    assert "kernel_ns_rocprof" not in r and "frac_kernel_rocprof" not in r
    h = r["rocprof_historical"]
    assert h["kernel_ns"] == 4000 and h["profiled_csrc_digest"] == "0" * 16 and h["current_csrc_digest"] == cur
    # No digest at all (a profile written before digests existed) is historical too.
    assert "rocprof_historical" in bench.rocprof_fields({"avg_ns": 1}, 1.0, 1.0, lambda v: v)


def test_kernel_digest_covers_sources_and_compiler_flags(tmp_path, monkeypatch):
    """The digest changes with any kernel source and with the Makefile, whose
    device-code flags (kernel-argument preloading among them) change the
    kernels' machine code as much as a source edit does."""
    import shutil

    import bench

    pkg = tmp_path / "soverign-grad_amd"
    shutil.copytree(ROOT / "soverign-grad_amd" / "csrc", pkg / "csrc")
    shutil.copy(ROOT / "soverign-grad_amd" / "Makefile", pkg / "Makefile")
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    d0 = bench.csrc_digest()
    assert d0 == bench.csrc_digest()
    mk = pkg / "Makefile"
    mk.write_text(mk.read_text().replace("-amdgpu-kernarg-preload-count=16", "-amdgpu-kernarg-preload-count=0"))
    d1 = bench.csrc_digest()
    assert d1 != d0
    src = pkg / "csrc" / "sgq_linear.hip"
    src.write_text(src.read_text() + "\n")
    assert bench.csrc_digest() not in (d0, d1)
    assert "-amdgpu-kernarg-preload-count=16" in (ROOT / "soverign-grad_amd" / "Makefile").read_text()


def _write_csv(path, header, rows):
    import csv

    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(header)
        w.writerows(rows)


def test_profile_summaries_from_rocprof_csvs(tmp_path):
    """The profiles/*.json records come from rocprofv3's CSVs: the dominant
    kernel's durations (graph dispatches after the eager ones) and its HBM
    bytes per launch scaled by the calibration copy, stamped with the digest
    of the kernel sources."""
    import bench

    gemv = "void sgq::(anonymous namespace)::k_gemv<4, 1, 4, 4, true, 1, 2, false, true>(sgq::(anonymous namespace)::GemvArgs)"
    trace = tmp_path / "t_kernel_trace.csv"
    hdr = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    rows = [["KERNEL_DISPATCH", 1, "__amd_rocclr_copyBuffer", 0, 5000]]
    durs = [9000, 9000, 4000, 4100, 4200, 3900]  # two eager dispatches, then four in graphs
    t = 10_000
    for i, d in enumerate(durs):
        rows.append(["KERNEL_DISPATCH", i + 2, gemv, t, t + d])
        t += d + 100
    _write_csv(trace, hdr, rows)
    r = bench.summarize_trace(str(trace), "c2", 2, "profiles/x.md")
    assert r["kernel"] == "k_gemv<4,1,4,4,true,1,2,false,true>"
    assert r["dispatches"] == 6 and r["graph_replay_dispatches"] == 4
    assert r["avg_ns_graph_replays"] == 4050 and r["median_ns_graph_replays"] == 4050
    assert r["avg_ns_all_dispatches"] == round(sum(durs) / 6) and r["min_ns"] == 3900
    assert r["csrc_digest"] == bench.csrc_digest()

    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    # The 64 MiB copy reads as half its bytes on FETCH_SIZE and in full on WRITE_SIZE.
    _write_csv(fetch, hdr, [[1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 32768.0],
                            [2, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 100.0],
                            [3, gemv, "FETCH_SIZE", 4400.0], [4, gemv, "FETCH_SIZE", 4500.0],
                            [5, gemv, "FETCH_SIZE", 4467.5]])
    _write_csv(write, hdr, [[1, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 65536.0],
                            [3, gemv, "WRITE_SIZE", 16.0], [4, gemv, "WRITE_SIZE", 16.0]])
    r = bench.summarize_traffic(str(fetch), str(write), "c2", "profiles/y.md")
    assert r["fetch_scale"] == 2.0 and r["write_scale"] == 1.0
    assert r["fetch_bytes"] == 4467.5 * 2 * 1024 and r["write_bytes"] == 16 * 1024
    assert r["hbm_bytes_per_launch"] == r["fetch_bytes"] + r["write_bytes"]
    assert r["csrc_digest"] == bench.csrc_digest() and r["kernel"] == "k_gemv<4,1,4,4,true,1,2,false,true>"
