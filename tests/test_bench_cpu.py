"""bench.py's CPU-side pieces: its FLOP convention agrees with the oracle's
pair count, its CPU baseline runs, and --gpus > 1 is refused."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


@pytest.mark.parametrize("sq,sk,causal,window", [(4096, 4096, True, -1), (1, 32768, False, -1), (4, 32768, False, -1),
                                                 (16384, 16384, False, 4096), (300, 100, True, 16),
                                                 (100, 300, True, 7), (333, 222, False, 5)])
def test_pair_count_matches_oracle(oracle_lib, sq, sk, causal, window):
    import bench

    assert bench.valid_pairs(sq, sk, causal, window) == oracle_lib.valid_pairs(sq, sk, causal, window)


def test_rope_interleaved_matches_oracle(oracle_lib):
    import numpy as np
    import torch

    import bench

    cos, sin = bench.rope_tables(40, 64)
    x = torch.randn(1, 2, 40, 64)
    got = bench.rope_interleaved(x, cos, sin)
    ref = oracle_lib.rope(x.numpy(), cos.numpy(), sin.numpy(), round_f16=False)
    np.testing.assert_allclose(got.numpy(), ref, atol=1e-6)


def test_cpu_baselines_small(oracle_lib):
    import bench

    wl = bench.Workload("f16", 1, 4, 2, 256, 256, 64, True, -1, True, 0, 1.0, "fa_fwd_f16_pp<64>")
    host = bench.cpu_inputs(wl)
    r, ref = bench.cpu_oracle_baseline(wl, host, budget_s=0.5)
    assert r["value"] > 0 and r["cores"] >= 1 and r["kind"] == "port"
    assert ref.shape[0] == 1 and ref.shape[1] % (wl.hq // wl.hkv) == 0 and ref.shape[2:] == (wl.sq, wl.d)
    r = bench.cpu_sdpa_baseline(wl, host, budget_s=0.5)
    assert r["value"] > 0 and r["cores"] >= 1


def test_sample_parity(oracle_lib):
    """sample_parity compares the sample's query heads (batch-major) of the
    step's output with the oracle's: the oracle's own output passes, a planted
    error in one element of the sample fails, and rows past the sample are not
    read."""
    import torch

    import bench

    wl = bench.Workload("f16", 2, 4, 2, 64, 64, 32, True, -1, False, 0, 1.0, "fa_fwd_f16_pp<32>")
    q, k, v, _, _ = bench.cpu_inputs(wl)
    full = oracle_lib.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=True)
    ref = full.reshape(1, 8, 64, 32)[:, :6]
    out = torch.from_numpy(full).half()
    assert bench.sample_parity(wl, out, ref)["ok"]
    bad = out.clone()
    bad.view(1, 8, 64, 32)[0, 5, 17, 3] += 0.01
    r = bench.sample_parity(wl, bad, ref)
    assert not r["ok"] and abs(r["max_abs"] - 0.01) < 1e-3
    past = out.clone()
    past.view(1, 8, 64, 32)[0, 7] = 5.0
    assert bench.sample_parity(wl, past, ref)["ok"]


def test_io_bytes_and_flops():
    import bench

    wl = bench.WORKLOADS["fp16_decode_b16_h32_kv8_sq1_sk32768_d128"]
    # Q + O (16*32*1*128 fp16 each) + K + V (16*8*32768*128 fp16 each)
    assert wl.io_bytes == 2 * 16 * 32 * 128 * 2 + 2 * 16 * 8 * 32768 * 128 * 2
    head = bench.WORKLOADS[bench.DEFAULT]
    assert head.flops == 4 * 4 * 32 * (4096 * 4097 // 2) * 128


def test_profiled_traffic_parses(tmp_path, monkeypatch):
    import bench

    wl = bench.WORKLOADS[bench.DEFAULT]
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    assert bench.profiled_traffic(bench.DEFAULT, wl) is None
    (tmp_path / "profiles").mkdir()
    # rocprofv3's kernel name "fa_fwd_f16_pp<128, true>" -> file-name stem
    assert wl.kernel == "fa_fwd_f16_pp<128, true>"
    (tmp_path / "profiles" / f"fa_fwd_f16_pp_128_true__{bench.DEFAULT}.md").write_text(
        "# x\n\ntraffic_bytes_per_launch: 123456\n")
    assert bench.profiled_traffic(bench.DEFAULT, wl) == 123456


def test_every_profiled_workload_has_a_summary():
    """Each bench workload whose traffic is reported reads a committed
    rocprofv3 summary named after its kernel; a renamed kernel instantiation
    must come with a renamed summary."""
    import bench

    for name in [bench.DEFAULT] + bench.SECONDARY:
        if name == "fp16_mha_b1_h8_s512_d64":
            continue
        assert bench.profiled_traffic(name, bench.WORKLOADS[name]) is not None, name


def test_pmc_summary(tmp_path, capsys):
    import bench

    d = tmp_path / "run"
    d.mkdir()
    (d / "run_counter_collection.csv").write_text(
        '"Kernel_Name","Counter_Name","Counter_Value"\n"k1","FETCH_SIZE",10.0\n"k1","FETCH_SIZE",30.0\n')
    assert bench.pmc_summary(str(tmp_path)) == 0
    out = capsys.readouterr().out
    assert "FETCH_SIZE" in out and "dispatches=2" in out and "20.0" in out


def test_pmc_derived_lds_and_wait(tmp_path):
    import bench

    mean = {("k", "SQ_LDS_IDX_ACTIVE"): 512.0, ("k", "GRBM_GUI_ACTIVE"): 8 * 4.0,
            ("k", "SQ_WAIT_ANY"): 30.0, ("k", "SQ_WAVE_CYCLES"): 120.0}
    (line,) = bench.pmc_derived(str(tmp_path), mean)
    # 512 LDS-busy cycles over 256 CUs x 4 cycles per XCD; 30 of 120 wave quad-cycles waiting
    assert "lds_util=0.5000" in line and "wait=0.2500" in line


def test_multi_gpu_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_trace_steps_splits_kernels_and_gaps(tmp_path, capsys):
    """bench.py --trace-steps on a synthetic kernel trace: two steps of a
    5 us pre-pass and a 100 us main kernel with 2 us and 3 us gaps."""
    import bench

    rows = ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    t = 0
    for _ in range(3):
        rows.append(f"rope_rotate_rows,{t},{t + 5000}")
        rows.append(f'"void rdna_amd::(anonymous namespace)::fa_fwd_f16_pp<128, true>(p)",{t + 7000},{t + 107000}')
        t += 110000
    (tmp_path / "run_kernel_trace.csv").write_text("\n".join(rows) + "\n")
    assert bench.trace_steps(str(tmp_path), "fa_fwd_f16_pp<128") == 0
    out = capsys.readouterr().out
    assert "steps=2 mean_step_us=110.00 gaps_us=5.00" in out
    assert "fa_fwd_f16_pp<128, true>" in out and "per_step_us=   100.00" in out
