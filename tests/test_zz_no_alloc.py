"""tm_adamw_step_noalloc (the allocation-free variant of tm_adamw_step) against tm_adamw_step,
through the C ABI: two calls in a row, the second over a smaller list, each bit for bit equal
to the workspace entry point's result on the same inputs. Also its argument checks."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests import _helpers as H

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import torchure_amd

    torchure_amd._native.lib()  # fail loudly if the HIP library is missing
    yield


def _call_both(shapes, seed):
    """The same clipped step through tm_adamw_step (the optimizer's own launch, workspace
    passed in) and through tm_adamw_step_noalloc on an identical copy; returns both sets."""
    import torchure_amd as ta
    from torchure_amd import _native

    host = H.make_host_set(shapes, seed=seed, grad_std=0.02)
    pa, wa, oa = H.device_setup(host, DEV)
    pb, wb, ob = H.device_setup(host, DEV)
    ta.clip_grad_norm(pa, None, 1.0)
    for launch in oa.plan_step(oa._pending[0], {id(p) for p in pa}):
        launch()
    oa._pending = None
    ta.clip_grad_norm(pb, None, 1.0)
    coef = ob._pending[0]
    launches = ob.plan_step(coef, {id(p) for p in pb})
    assert len(launches) == 1
    sl = launches[0]
    print(f"noalloc: {sl.n} tensors, {sl.n_chunks} chunks", flush=True)
    rc = _native.lib().tm_adamw_step_noalloc(sl.d_rows.data_ptr(), sl.n, sl.chunks.data_ptr(), sl.n_chunks,
                                             sl.chunk_elems, sl.groups_c, sl.n_groups, coef.data_ptr(),
                                             _native.stream_handle(DEV))
    _native.check(rc, "tm_adamw_step_noalloc")
    ob._pending = None
    torch.cuda.synchronize()
    return (pa, wa, oa), (pb, wb, ob)


def _assert_same(a, b):
    (pa, wa, oa), (pb, wb, ob) = a, b
    for x, y, u, v in zip(pa, pb, wa, wb):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))
        for k in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(oa.state[x][k].view(torch.int32), ob.state[y][k].view(torch.int32))


def test_noalloc_step_equals_workspace_step_twice():
    big = [(512, 300), (1031,), (77, 45), (4096,), (33,), (2048, 64)]
    _assert_same(*_call_both(big, 91))
    _assert_same(*_call_both(big[:3], 92))  # the second call, over a smaller list


def test_noalloc_step_argument_checks():
    from torchure_amd import _native

    lib = _native.lib()
    hyper = _native.hyper_array([(3e-4, 0.9, 0.95, 0.1, 1e-8)])
    fake = ctypes.c_void_p(0x1000)
    too_many = _native.TM_NOALLOC_MAX_TENSORS + 1
    assert lib.tm_adamw_step_noalloc(fake, too_many, fake, too_many, 2048, hyper, 1, None, None) < 0
    assert b"at most" in lib.tm_last_error()
    assert lib.tm_adamw_step_noalloc(fake, 1, fake, 1, 2048, hyper, 0, None, None) < 0
    assert b"n_groups" in lib.tm_last_error()
    assert lib.tm_adamw_step_noalloc(None, 0, None, 0, 2048, hyper, 1, None, None) == _native.TM_OK
