"""The bench's counter reducers on synthetic rocprofv3 output (CPU only).

The committed profiles are reduced from rocprofv3 csv counter files by
``bench.py --mfma-from``, ``--sq-from`` and ``--train-traffic-from``; these
tests feed them small hand-written counter files whose reductions are known,
and check the refusal of more than one GPU."""
import csv
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
          "Start_Timestamp", "End_Timestamp"]


def write_run(d: Path, rows):
    """rows: (dispatch, kernel, counter, value, ns) -> d/x/run_counter_collection.csv"""
    (d / "x").mkdir(parents=True)
    with open(d / "x" / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, FIELDS)
        w.writeheader()
        for did, k, c, v, ns in rows:
            w.writerow({"Dispatch_Id": did, "Kernel_Name": k, "Counter_Name": c,
                        "Counter_Value": v, "Start_Timestamp": 1000,
                        "End_Timestamp": 1000 + ns})


F32 = "void gdn2::fwd_state<float, 64, 128, 2, 4, 2, 0>(gdn2::StateArgs<float>)"
BF = "void gdn2::fwd_prep<__bf16, float, 128, 128, __bf16, 0>(gdn2::PrepArgs<__bf16>)"


def test_mfma_from_counts_split_products_a_third(tmp_path, capsys):
    # a float32 kernel with 300 bf16 MOPS (split products: 100 fp32-equivalent) and
    # 50 fp32 MOPS, over 2 us; counters arrive per XCD instance and are summed
    rows = [(7, F32, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 150.0, 2000),
            (7, F32, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 150.0, 2000),
            (7, F32, "SQ_INSTS_VALU_MFMA_MOPS_F32", 50.0, 2000),
            (7, F32, "SQ_VALU_MFMA_BUSY_CYCLES", 1024.0 * 10, 2000),
            (7, F32, "GRBM_GUI_ACTIVE", 8 * 40.0, 2000),
            (9, BF, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 10.0, 1000)]
    write_run(tmp_path, rows)
    out = bench.mfma_from(tmp_path)
    capsys.readouterr()
    r = out["fwd_state (fp32)"]
    assert r["bf16_mfma_flops"] == 512 * 300 and r["f32_mfma_flops"] == 512 * 50
    assert r["mfma_flops"] == pytest.approx(512 * (50 + 300 / 3))
    assert r["tflops"] == pytest.approx(512 * 150 / 2000 / 1e3)
    assert r["mfma_busy"] == pytest.approx(10 / 40)        # per-XCD GRBM x 1024 SIMDs
    b = out["fwd_prep (bf16)"]
    assert b["mfma_flops"] == 512 * 10                       # bf16 kernels: counted in full
    assert b["frac_of_peak"] == pytest.approx(512 * 10 / 1000 / 1e3 / 2516.6)


def test_sq_from_takes_last_dispatch_and_merges_passes(tmp_path, capsys):
    a, b = tmp_path / "a", tmp_path / "b"
    # pass A: the kernel twice; only the second dispatch (id 5) counts
    write_run(a, [(2, F32, "SQ_WAVE_CYCLES", 999.0, 1), (2, F32, "SQ_WAIT_ANY", 999.0, 1),
                  (5, F32, "SQ_WAVES", 4.0, 1), (5, F32, "SQ_WAVE_CYCLES", 200.0, 1),
                  (5, F32, "SQ_WAVE_CYCLES", 200.0, 1), (5, F32, "SQ_WAIT_ANY", 100.0, 1),
                  (5, F32, "SQ_WAIT_INST_ANY", 60.0, 1), (5, F32, "SQ_ACTIVE_INST_ANY", 240.0, 1),
                  (5, F32, "SQ_ACTIVE_INST_VALU", 40.0, 1)])
    # pass B: instruction counts of the same kernel (its own dispatch ids)
    write_run(b, [(3, F32, "SQ_WAVES", 4.0, 1), (3, F32, "SQ_INSTS_VALU", 400.0, 1),
                  (3, F32, "SQ_INSTS_LDS", 8.0, 1), (3, F32, "SQ_LDS_BANK_CONFLICT", 12.0, 1)])
    out = bench.sq_from([a, b])
    capsys.readouterr()
    r = out["fwd_state (fp32)"]
    assert r["wait_any"] == pytest.approx(100 / 400)
    assert r["wait_inst_any"] == pytest.approx(60 / 400)
    assert r["active_any"] == pytest.approx(240 / 400)
    assert r["active_valu"] == pytest.approx(40 / 400)
    assert r["valu_per_wave"] == 100 and r["lds_per_wave"] == 2
    assert r["lds_bank_conflict_per_wave"] == 3 and r["waves"] == 4


def test_counter_means_refuse_two_runs_in_one_directory(tmp_path):
    write_run(tmp_path / "r1", [(1, F32, "FETCH_SIZE", 1.0, 1)])
    write_run(tmp_path / "r2", [(1, F32, "FETCH_SIZE", 1.0, 1)])
    with pytest.raises(SystemExit):
        bench._counter_means(tmp_path, "FETCH_SIZE")


def test_counter_means_calibration_is_the_last_dispatch(tmp_path):
    copy = "copy_kernel"
    write_run(tmp_path, [(1, F32, "FETCH_SIZE", 10.0, 1), (2, F32, "FETCH_SIZE", 30.0, 1),
                         (3, copy, "FETCH_SIZE", 512.0, 1), (3, copy, "FETCH_SIZE", 512.0, 1)])
    means, last = bench._counter_means(tmp_path, "FETCH_SIZE")
    assert means[F32] == 20.0 and last == 1024.0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
    assert not r.stdout.strip()
