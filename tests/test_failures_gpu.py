"""Failure handling of the token loop on the GPU (the reference's convention it replaces is
assert + log + silent return, e.g. MatrixDX11_Functions.h:92-120, where a failed allocation or
a missing shader leaves the previous contents in place).

Here every failure surfaces as an FMLH_E_* status with a message, and a token loop that failed
never hands out stale tokens or logits: readers refuse until the next prefill.  The failures are
forced from the host with the FMLH_FAULT hook (alloc:N / launch:N, re-armed at each fmlh_init):
the sweeps below fail every allocation and every launch check of engine creation, prefill and
decode in turn, on the persistent, graph and relay decode paths (relay: c2's shape) and through
the fused prefill split over two streams (c3's 64 sequences), and check
after each that the error names the hook, that nothing stale is readable and that the same
engine then decodes the oracle's tokens.

Each sweep runs in a child process so that the hook and fmlh_shutdown do not touch the test
process's own library state.  No kernel is made to fail on the device: an injected launch
failure is reported after a normal launch (or instead of the persistent launch).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SWEEP = r"""
import os, sys
import numpy as np
sys.path.insert(0, {root!r})
import freeml_amd as fh
import oracle
from freeml_amd import synth

kind, path = sys.argv[1], sys.argv[2]
if path == "graph":
    os.environ["FMLH_DECODE"] = "graph"
if path == "relay":
    os.environ["FMLH_RELAY"] = "1"
# the relay kernel is compiled for c2's width; c3's 64 sequences take the fused prefill on two
# streams
cfg = "c2" if path == "relay" else "c3" if path == "prefill_parts" else "c1"
B = synth.CONFIGS[cfg]["batch"] if path == "prefill_parts" else 1
w = synth.make_weights(synth.CONFIGS[cfg]["shape"], 0)
p = synth.prompts_for(cfg)
t_ref, l_ref = oracle.OracleModel(w).greedy(p[0], 12, cached=True)
fired = 0
for n in range(1, 400):
    os.environ["FMLH_FAULT"] = f"{{kind}}:{{n}}"
    fh.init(0)  # re-arms the hook
    m = None
    try:
        m = fh.NanoLLM(w, max_batch=B)
        m.prefill(p)
        m.decode(6)
        m.decode(5)
        toks, lg = m.tokens(), m.logits()
    except fh.FreeMLHipError as e:
        assert "FMLH_FAULT" in str(e), f"{{kind}}:{{n}}: unexpected error {{e}}"
        fired += 1
        if m is not None:
            for read in (m.logits, m.tokens):
                try:
                    read()
                except fh.FreeMLHipError:
                    continue
                raise AssertionError(f"{{kind}}:{{n}}: state readable after a failure")
            os.environ.pop("FMLH_FAULT")
            fh.init(0)  # disarm, then the same engine must work again
            toks, lg = m.generate(p, 12, with_logits=True)
            assert np.array_equal(toks[0], t_ref), f"{{kind}}:{{n}}: wrong tokens after recovery"
            err = np.max(np.abs(lg[0] - l_ref)) / np.max(np.abs(l_ref))
            assert err <= 1e-4, f"{{kind}}:{{n}}: logits off by {{err}} after recovery"
            m.close()
        print(f"{{kind}}:{{n}} failed cleanly", flush=True)
        continue
    # the hook fired nowhere: every event of the sequence has been covered
    assert np.array_equal(toks[0], t_ref[:12]), "unfaulted run differs from the oracle"
    # The relay path, unless the runtime refused the cooperative launch (ROCm gives the
    # device's cooperative-launch resource to one process at a time: a parent process that
    # launched a cooperative kernel first keeps it) and the engine fell back, as it must.
    got, last = m.decode_path(1)[0], fh.lib().fmlh_last_error().decode(errors="replace")
    print(f"final decode path: {{got}}", flush=True)
    if path == "relay":
        assert got == "relay" or "cooperative launch refused" in last, (got, last)
    m.close()
    break
else:
    raise AssertionError("sweep did not reach a run without a fault")
print(f"SWEEP_OK {{kind}} {{path}}: {{fired}} injected failures", flush=True)
"""

SHUTDOWN = r"""
import sys
import numpy as np
sys.path.insert(0, {root!r})
import freeml_amd as fh
from freeml_amd import synth

fh.init(0)
w = synth.make_weights(synth.CONFIGS["c1"]["shape"], 0)
p = synth.prompts_for("c1")
m = fh.NanoLLM(w, max_batch=1)
t0, _ = m.generate(p, 8)
handle = m.h
fh.call("fmlh_shutdown")
for fn, args in (("fmlh_synchronize", ()), ("fmlh_nanollm_destroy", (handle,))):
    try:
        fh.call(fn, *args)
    except fh.FreeMLHipError as e:
        print(fn, "refused:", e, flush=True)
        continue
    raise AssertionError(fn + " succeeded after fmlh_shutdown")
m.h = None  # released by the shutdown
fh.init(0)  # starts the library again
m2 = fh.NanoLLM(w, max_batch=1)
t1, _ = m2.generate(p, 8)
assert np.array_equal(t0, t1)
print("SHUTDOWN_OK", flush=True)
"""


def _run(script, *args, timeout=240):
    env = dict(os.environ)
    env.pop("FMLH_FAULT", None)
    r = subprocess.run([sys.executable, "-u", "-c", script.format(root=ROOT), *args], env=env,
                       capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0, f"child exited with {r.returncode}"
    return r.stdout


@pytest.mark.parametrize("path", ["persistent", "graph", "relay", "prefill_parts"])
@pytest.mark.parametrize("kind", ["alloc", "launch"])
def test_every_forced_failure_surfaces_and_leaves_nothing_stale(kind, path):
    out = _run(SWEEP, kind, path)
    assert f"SWEEP_OK {kind} {path}" in out


def test_shutdown_releases_engines_and_refuses_stale_handles():
    assert "SHUTDOWN_OK" in _run(SHUTDOWN)
