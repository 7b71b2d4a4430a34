"""The step timeline (plamo_timeline, `make timeline`): device timestamps of replayed decode
steps are consistent with the step's dependency chain, and the normal library refuses it."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_normal_library_has_no_timeline():
    import plamo_hip
    with pytest.raises(plamo_hip.PlamoError, match="without the step timeline"):
        plamo_hip.timeline()


def test_timeline_of_replayed_steps():
    from plamo_hip import native
    if not os.path.exists(native.TIMELINE_LIB_PATH):
        pytest.skip("timeline library not built (make -C plamo3-0.8b-runtime_amd timeline)")
    # a child process: this one holds the normal library
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--timeline"], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    import json
    r = json.loads(out.stdout.strip().splitlines()[-1])
    print(json.dumps(r), flush=True)
    k = r["kernels"]
    # 16 layers of qkv, attention, o, gate_up, down, then the LM head and its merge
    assert {n: k[n]["launches_per_step"] for n in ("qkv", "attention", "o", "gate_up", "down")} == \
        {n: 16 for n in ("qkv", "attention", "o", "gate_up", "down")}
    assert k["head"]["launches_per_step"] == 1 and k["head_merge"]["launches_per_step"] == 1
    assert r["kernels_per_step"] == 82 and "step_begin" not in k
    # each kernel depends on the one before it: its first workgroup starts only after the
    # previous kernel's last workgroup ended (one 10 ns tick of slack)
    assert r["gap_min_us"] >= -0.01
    # the stamps are in 100 MHz ticks: the step span they give fits inside the HIP-event time
    # of the same replays (which adds the graph launch) and covers most of it
    assert 0.6 * r["event_ms_per_step"] * 1000 <= r["step_span_us"] <= 1.02 * r["event_ms_per_step"] * 1000
