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


def test_noalloc_step_captured_in_a_hip_graph():
    """The allocation-free step is what a caller under HIP graph capture can launch: captured in
    a torch.cuda.CUDAGraph and replayed three times, with eager work and synchronisations
    between the replays, it leaves after every replay the state of as many eager
    tm_adamw_step_noalloc calls on an identical copy, bit for bit (each replay advances the
    device-side step counters, so the bias corrections change from replay to replay)."""
    from torchure_amd import _native

    lib = _native.lib()
    shapes = [(512, 300), (1031,), (77, 45), (4096,), (33,)]
    host = H.make_host_set(shapes, seed=95, grad_std=0.02)
    graph_set = H.device_setup(host, DEV)
    eager_set = H.device_setup(host, DEV)
    warm_set = H.device_setup(host, DEV)

    def launch(sl):
        rc = lib.tm_adamw_step_noalloc(sl.d_rows.data_ptr(), sl.n, sl.chunks.data_ptr(), sl.n_chunks,
                                       sl.chunk_elems, sl.groups_c, sl.n_groups, None,
                                       _native.stream_handle(DEV))
        _native.check(rc, "tm_adamw_step_noalloc")

    plans = [opt.plan_step(None, set()) for _, _, opt in (graph_set, eager_set, warm_set)]
    assert all(len(p) == 1 for p in plans)
    graph_launch, eager_launch, warm_launch = (p[0] for p in plans)
    launch(warm_launch)  # the first call on the device looks up the static scratch, outside capture
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            launch(graph_launch)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _assert_same(graph_set, H.device_setup(host, DEV))  # capturing ran nothing

    for k in range(3):
        print(f"replay {k}", flush=True)
        g.replay()
        launch(eager_launch)
        torch.cuda.synchronize()
        assert torch.randn(4096, device=DEV).abs().sum().item() > 0  # eager work between replays
        _assert_same(graph_set, eager_set)
        assert float(graph_set[2].state[graph_set[0][0]]["step"].item()) == 1000.0 + k + 1


def test_noalloc_step_on_views_off_their_1kib_boundaries():
    """The same comparison on tensors that are views of pooled buffers starting 4 to 252
    elements past a 1 KiB boundary, with lengths that make the update's shifted slice grid
    wrap its last elements into the first slice: tm_adamw_step_noalloc and tm_adamw_step give
    the same bits on two identical copies."""
    import torchure_amd as ta
    from torchure_amd import _native

    specs = [(n, dict(p=ph, m=ph, v=ph, g=ph, w=ph), False)
             for ph in (4, 128, 252) for n in (5, 255, 16384 - ph + 1, 16384, 3 * 16384 + 130)]
    specs.append((2 * 16384 + 9, dict(p=64, m=128, v=128), False))
    a = H.views_at_phases(specs, DEV, seed=97)
    b = H.views_at_phases(specs, DEV, seed=97)
    print(f"noalloc views: {len(specs)} tensors", flush=True)
    (_, pa, wa, oa, _), (_, pb, wb, ob, _) = a, b
    ta.clip_grad_norm(pa, None, 0.05)
    for launch in oa.plan_step(oa._pending[0], {id(p) for p in pa}):
        launch()
    oa._pending = None
    ta.clip_grad_norm(pb, None, 0.05)
    coef = ob._pending[0]
    (sl,) = ob.plan_step(coef, {id(p) for p in pb})
    rc = _native.lib().tm_adamw_step_noalloc(sl.d_rows.data_ptr(), sl.n, sl.chunks.data_ptr(), sl.n_chunks,
                                             sl.chunk_elems, sl.groups_c, sl.n_groups, coef.data_ptr(),
                                             _native.stream_handle(DEV))
    _native.check(rc, "tm_adamw_step_noalloc")
    ob._pending = None
    torch.cuda.synchronize()
    _assert_same((pa, wa, oa), (pb, wb, ob))
