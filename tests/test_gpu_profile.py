"""BROLM_PROFILE stage timer (reference include/brolm/detail/profile.h:19-69)
on HIP events, and brotensor::shutdown().  Each case runs in a child process:
the gate is read once per process, and shutdown ends the runtime."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent

CHILD = r"""
import json, sys, time
sys.path.insert(0, {root!r}); sys.path.insert(0, {tests!r})
import numpy as np
import brolm_amd as ba, oracle
path = {path!r}
ba.init()
m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(path)); m.load_weights(path); m.allocate_cache(64)
om = oracle.Model(path); om.allocate_cache(64)
prompt = [3, 1, 4, 1, 5, 9, 2, 6]
ba.profile_reset()
t0 = time.perf_counter()
a = m.forward_last(prompt)
tok = int(a.argmax())
steps = [m.forward_last([tok])]
wall_ns = (time.perf_counter() - t0) * 1e9
b = om.forward(prompt, last_only=True)[0]
c = om.forward([tok], last_only=True)[0]
st = ba.profile_stages()
ba.profile_report()
diff = float(max(np.abs(a - b).max(), np.abs(steps[0] - c).max()))
# shutdown with the model still open, then close it, then a fresh runtime
ba.shutdown()
m.close()
ba.init()
m2 = ba.Qwen3Model(ba.Qwen3Config.from_gguf(path)); m2.load_weights(path); m2.allocate_cache(64)
d = float(np.abs(m2.forward_last(prompt) - b).max())
m2.close()
ba.shutdown()
print("RESULT " + json.dumps(dict(stages=st, wall_ns=wall_ns, diff=diff, diff2=d)), flush=True)
"""


def _child(small_gguf, env_extra):
    env = dict(os.environ, **env_extra)
    code = CHILD.format(root=str(ROOT), tests=str(ROOT / "tests"), path=str(small_gguf))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0, r.stderr[-2000:]
    line = [l for l in r.stdout.splitlines() if l.startswith("RESULT ")][-1]
    return json.loads(line[len("RESULT "):]), r.stderr


@pytest.mark.timeout(300)
def test_stage_timer_on_events(small_gguf):
    res, err = _child(small_gguf, {"BROLM_PROFILE": "1"})
    st = res["stages"]
    for stage in ("embed", "qkv_proj", "attention", "o_proj", "mlp_proj", "lm_head"):
        assert stage in st and st[stage][1] > 0 and st[stage][0] > 0, stage
    # one prefill + one single-token step, each through every layer's stages
    assert st["qkv_proj"][1] == st["attention"][1] == 2 * 2
    # device time between events: the stages never add up to more than the
    # host's wall time around the work
    assert sum(ns for ns, _ in st.values()) <= res["wall_ns"]
    assert "BROLM_PROFILE" in err and "attention" in err
    assert res["diff"] <= 2e-2 and res["diff2"] <= 2e-2


@pytest.mark.timeout(300)
def test_shutdown_then_reinit_without_profiling(small_gguf):
    res, _ = _child(small_gguf, {"BROLM_PROFILE": "0"})
    assert res["stages"] == {}
    assert res["diff"] <= 2e-2 and res["diff2"] <= 2e-2
