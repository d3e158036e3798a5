"""Handles left open at interpreter exit: the package's atexit hook closes
sessions, models and contexts (in that order) while the HIP runtime is intact,
so nothing is left for the runtime's own exit-time teardown.  The child
process decodes through the persistent kernel (mapped host words, its own
stream) and exits without closing anything."""
import os
import subprocess
import sys
import textwrap

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_open_handles_are_closed_at_exit():
    script = textwrap.dedent("""
        import atexit, sys
        # registered before the package's hook, so it runs after it (LIFO)
        atexit.register(lambda: print("still open after close_all:",
                                      sum(1 for o in sys.modules["alpaca_amd.model"]._LIVE if o.handle), flush=True))
        import numpy as np
        from alpaca_amd import synth, model as M
        spec = synth.TINY
        ctx = M.HIPContext(0)
        m = M.HIPLlamaModel(ctx, spec.config, synth.build_weights(spec))
        s = m.make_session(capacity=96)
        t = int(np.argmax(s.forward(synth.prompt_tokens(spec, 20))))
        s.decode_greedy(t, 4, lambda x: True)
        live = sorted(o._kind for o in M._LIVE)
        print("live before exit:", live, flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", script], cwd=ROOT, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "live before exit: ['context', 'model', 'session']" in r.stdout, r.stdout
    assert "still open after close_all: 0" in r.stdout, r.stdout
