"""CPU checks of bench.py's host logic: the roofline traffic it reads from
the committed rocprofv3 summary, and the one-GPU refusal."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_traffic_comes_from_the_committed_profile():
    t = bench.profiled_traffic()
    assert isinstance(t, int)
    shapes = bench.step_shapes()
    algo = sum(bench.algo_bytes(o, i, bench.H.Q4_0, 1) for _, o, i in shapes)
    # The counters read the packed weights once: within a few percent of the algorithmic bytes.
    assert 0.9 * algo <= t <= 1.1 * algo


def test_traffic_parser_reads_the_named_row(tmp_path):
    p = tmp_path / "t.md"
    p.write_text("| kernel | dispatches | HBM bytes (scaled) |\n|---|---|---|\n| `k<1>` | 3 | 1,234 |\n"
                 "| `k<2>` | 3 | 99 |\n")
    assert bench.profiled_traffic("k<2>", str(p)) == 99
    assert bench.profiled_traffic("k<3>", str(p)) is None
    assert bench.profiled_traffic("k<1>", str(tmp_path / "missing.md")) is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_weight_bytes_of_each_type():
    assert bench.weight_bytes_of(4, 64, bench.H.F32) == 4 * 4 * 64
    assert bench.weight_bytes_of(4, 64, bench.H.Q8_0) == 4 * 64 + 4 * 4 * 2
    assert bench.weight_bytes_of(4, 64, bench.H.Q4_0) == 4 * 32 + 4 * 4 * 2


def test_final_line_stays_compact():
    """The driver parses the last stdout line from a bounded tail: the line
    built from a full record of a default run (decode id lists, the
    per-shape table, sampling detail) must stay under bench.LINE_LIMIT and
    keep the contract's fields."""
    import json

    with open(os.path.join(ROOT, "tests", "data", "bench_full_record.json")) as f:
        full = json.load(f)
    full["decode_tolerance_mode"] = {k: {"decode_tok_s": 2345.6, "frac_of_roofline": 0.0961,
                                         "ids_match_first64": True, "ids_match_reference": False,
                                         "max_rel_logit_err": 1.23e-6, "extra": list(range(500))}
                                     for k in full["decode"]}
    line = bench.compact_line(full, os.path.join(ROOT, "gpurun_out", "bench_full.json"))
    text = json.dumps(line)
    assert len(text) < bench.LINE_LIMIT, len(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype", "config",
              "roofline", "cpu_baseline", "decode", "prefill_gemm_c5", "targets_qwen25_pct_hbm_peak"):
        assert k in line, k
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in line["roofline"], k
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in line["cpu_baseline"], k
    c4 = line["decode"]["c4_qwen25_05b_q4_0"]
    assert c4["ids_match_reference"] is True
    ids = full["decode"]["c4_qwen25_05b_q4_0"]["generate_json"]["generated_ids"]
    assert c4["generated_ids_sha256"] == bench.ids_sha256(ids)
    assert "extra" not in line["decode_tolerance_mode"]["c4_qwen25_05b_q4_0"]
    assert line["full_record"] == os.path.join("gpurun_out", "bench_full.json")
