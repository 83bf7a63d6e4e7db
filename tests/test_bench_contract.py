"""bench.py's command-line contract on the CPU: the workload list, the one-GPU rule, and the profile readers that feed
the JSON line's roofline fields."""
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=ROOT, timeout=120)
    assert r.returncode != 0
    assert "GPU" in r.stderr and r.stdout.strip() == ""


def test_profile_readers_parse_committed_summaries():
    for name in ("decode_attn_serving_b256_pmc_traffic.md", "decode_attn_saturated_b256_pmc_traffic.md",
                 "prefill_masked_b4_s10240_pmc_traffic.md", "kv_move_compaction_64seq_pmc_traffic.md",
                 "decode_attn_full_model_b64_pmc_traffic.md", "prefill_masked_bwd_b4_s10240_pmc_traffic.md"):
        t = bench.profiled_traffic(name)
        assert t is not None and t > 1e8, name
    u = bench.profiled_mfma_util("prefill_masked_b4_s10240_pmc_mfma.md")
    assert u is not None and 0.0 < u < 1.0
    assert bench.profiled_traffic("no_such_profile.md") is None


def test_every_workload_parses_with_defaults(monkeypatch):
    for wl in ("serving", "saturated", "full_model", "config1", "prefill", "prefill_bwd", "compaction", "packed",
               "code_step", "copy"):
        monkeypatch.setattr(sys, "argv", ["bench.py", "--workload", wl])
        a = bench.parse()
        assert a.workload == wl and a.gpus == 1 and a.steps > 0 and a.warmup >= 0
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    assert bench.parse().workload == "serving"
