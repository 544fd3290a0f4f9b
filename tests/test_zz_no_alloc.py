"""goi_step_n_noalloc, the entry point that allocates nothing, against goi_step_n through the C ABI.

Both launch the same kernels; the allocation-free one keeps the constraint rows in the library's static device array.
Two calls in a row (the second with fewer worlds, so stale rows of the first call lie beyond the second's tiles)
must each equal goi_step_n on the same input bit for bit, and a batch needing more rows than the array holds is
refused on the host with GOI_E_UNSUPPORTED before anything is launched.
"""
import ctypes
import importlib

import numpy as np
import pytest

from util import b2, leaf_mismatches, wd

torch = pytest.importorskip("torch")
step_mod = importlib.import_module("getting-over-it-rl_amd.box2d.step")
pytestmark = pytest.mark.gpu


def _first(state, n):
    return wd.from_leaves([np.ascontiguousarray(np.asarray(x)[:n]) for x in wd.leaves(state)])


def _call(fn, m, dev, s, dt, n_steps):
    view = b2.layout.state_view(dev)
    dm = step_mod.device_model(m, dev.contacts.pair.shape[-1], dev.contacts.pair.device, dev)
    cs = s.to_c()
    stream = torch.cuda.current_stream().cuda_stream
    return getattr(dm.L, fn)(dm.handle, ctypes.byref(view), ctypes.byref(cs), ctypes.c_float(np.float32(dt)),
                             ctypes.c_int32(n_steps), ctypes.c_void_p(stream), None)


@pytest.mark.parametrize("wpw,kernel", [(None, "generic"), ("8", "rig")])
def test_noalloc_equals_step_n_twice(monkeypatch, wpw, kernel):
    """The default wave size (1 world a wave at these batch sizes: the generic kernel) and 8 worlds a wave (the
    packed rig State then runs the instance compiled for the rig, the headline workload's kernel)."""
    if wpw is not None:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    s, m, st, cfg = b2.scenes.make_config(4, 1536)
    A = b2._abi
    for n, n_steps in ((1536, 3), (384, 2)):
        part = _first(st, n)
        want = b2.layout.to_device(part, "cuda")
        got = b2.layout.to_device(part, "cuda")
        A.check(_call("goi_step_n", m, want, s, cfg.dt, n_steps))
        A.check(_call("goi_step_n_noalloc", m, got, s, cfg.dt, n_steps))
        info = b2.last_launch()
        assert info["kernel"] == kernel and (wpw is None or info["worlds_per_wave"] == int(wpw)), info
        torch.cuda.synchronize()
        bad = leaf_mismatches(b2.layout.to_host(want), b2.layout.to_host(got))
        assert bad == [], (n, bad[:4])
        assert int(np.asarray(b2.layout.to_host(got).toi.events).sum()) > 0


def test_noalloc_refuses_a_batch_above_its_maximum():
    """The headline batch (16,384 rig worlds with 40 slots) needs (40 * 54 + 3 * 57) * (16,384 + 64) words of rows,
    more than the static array's 2^25: refused before anything runs."""
    s, m, st, cfg = b2.scenes.make_config(4, 16384)
    dev = b2.layout.to_device(st, "cuda")
    torch.cuda.synchronize()
    before = b2.layout.to_host(dev)
    A = b2._abi
    L = A.lib()
    assert _call("goi_step_n_noalloc", m, dev, s, cfg.dt, 1) == A.GOI_E_UNSUPPORTED
    assert b"static maximum" in L.goi_last_error()
    torch.cuda.synchronize()
    assert leaf_mismatches(before, b2.layout.to_host(dev)) == []
