"""Host logic of bench.py that needs no GPU: the other workloads' entries
collected from child processes (`other_configs`), including a child that
fails and one that gives no result in time."""
import json
import os
import subprocess
import sys
import types

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def child_line(name):
    line = {"metric": bench.METRIC if name != "qwen3" else "ms per text encode", "value": 1.5,
            "unit": "images/s", "ms_per_step": 10.0, "mfma_frac_step": 0.4,
            "config": {"workload": f"{name} workload", "hidden": 3072},
            "roofline": {"kernel": "k", "launch_ms": 0.1, "frac": 0.5, "achieved": 1.0},
            "kernels": [{"key": "a", "launch_ms": 0.1, "frac": 0.5, "flop_per_launch": 2.0}]}
    if name == "c5":
        line["parity"] = {"pass": True}
    return json.dumps(line)


def test_other_configs_collects_children(monkeypatch):
    calls = []

    def fake_run(cmd, capture_output, text, timeout):
        assert capture_output and text and timeout > 0
        calls.append(cmd)
        name = cmd[cmd.index("--config") + 1]
        if name == "c3":
            return subprocess.CompletedProcess(cmd, 1, "", "Traceback\nAssertionError: boom")
        if name == "c4":
            raise subprocess.TimeoutExpired(cmd, timeout)
        if name == "vae":
            return subprocess.CompletedProcess(cmd, 0, "no json here\n", "")
        return subprocess.CompletedProcess(cmd, 0, "progress\n" + child_line(name) + "\n", "")

    monkeypatch.setattr(bench.subprocess, "run", fake_run)
    out = bench.other_configs(types.SimpleNamespace(steps=3, warmup=1))
    assert list(out) == bench.OTHER_CONFIGS
    assert [c[c.index("--config") + 1] for c in calls] == bench.OTHER_CONFIGS
    for c in calls:
        assert "--no-cpu-baseline" in c
        assert c[c.index("--steps") + 1] == "3" and c[c.index("--warmup") + 1] == "1"
    assert out["c3"] == {"error": "exit status 1: AssertionError: boom"}
    assert out["c4"] == {"error": "no result within 150 s"}
    assert out["vae"]["error"].startswith("exit status 0")
    # the headline metric text is not repeated for the other Flux workloads
    assert "metric" not in out["c2"] and out["qwen3"]["metric"] == "ms per text encode"
    assert out["c2"]["workload"] == "c2 workload" and out["c2"]["ms_per_step"] == 10.0
    assert out["c2"]["roofline"] == {"kernel": "k", "launch_ms": 0.1, "frac": 0.5}
    assert out["c2"]["kernels"] == [{"key": "a", "launch_ms": 0.1, "frac": 0.5}]
    assert out["c5"]["parity"] == {"pass": True} and "parity" not in out["c2"]
