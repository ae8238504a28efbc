"""GPU parity of the chunked fused linear + cross-entropy (torchure/loss/fused_linear_ce.py).

Checks:
- the fused CE-row kernel vs an fp64 restatement on the same bf16 logits: per-row
  loss within 1e-6 relative, grad_logits = bf16(softmax - onehot) within 1 bf16 ulp;
  the in-register path (V <= 163,840), the two-read path (larger V) and the
  element-wise path (rows not 16-byte aligned) are all exercised;
- the whole op (forward + backward through autograd) vs the reference's own
  composition (torchure/loss/fused_linear_ce.py, same torch calls) on the same
  device: same GEMMs, so the loss agrees within 1e-5 relative and the grads
  within bf16 resolution;
- the reference's own test cases (tests/fused_linear_ce.py), against an unfused
  lm_head + F.cross_entropy at that test's bars, plus the trainer's own call (fp32 hidden
  under bf16 autocast, 4096-row chunks);
- the grad_W hand-over (one chunk, or two in one pass) bit for bit against torch's `+=` and
  `mul_`, and the whole chunk loop bit for bit for 1, 2, 3, 4 and 7 chunks;
- fp32 hidden under autocast, ignore_index values inside the vocabulary, non-contiguous
  inputs, the loss-only path and gradients for only one input.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from oracle.torch_composition import fused_linear_ce_reference
from tests import _helpers as H

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import torchure_amd

    torchure_amd._native.lib()
    yield


def _ce_rows(logits_bits: np.ndarray, labels: np.ndarray, ignore: int):
    from torchure_amd import _native

    rows, v = logits_bits.shape
    d_logits = torch.from_numpy(logits_bits.view(np.int16).copy()).to(DEV)
    d_labels = torch.from_numpy(labels.astype(np.int64)).to(DEV)
    d_loss = torch.empty(rows, dtype=torch.float32, device=DEV)
    rc = _native.lib().tm_ce_rows_bf16(d_logits.data_ptr(), v, d_labels.data_ptr(), rows, v, ignore,
                                       d_loss.data_ptr(), _native.stream_handle(DEV))
    _native.check(rc, "tm_ce_rows_bf16")
    torch.cuda.synchronize()
    return d_logits.cpu().numpy().view(np.uint16), d_loss.cpu().numpy()


@pytest.mark.parametrize("vocab", [4096, 1001, 151936, 200000])
def test_ce_rows_kernel_vs_fp64(vocab):
    r = H.rng(vocab)
    rows = 37
    x = (r.standard_normal((rows, vocab)) * 3.0).astype(np.float32)
    bits = oracle.bf16_rne(x).reshape(rows, vocab)
    labels = r.integers(0, vocab, rows)
    labels[[3, 17]] = -100
    grad_bits, loss = _ce_rows(bits, labels, -100)
    xd = oracle.bf16_to_f32(bits).reshape(rows, vocab).astype(np.float64)
    mx = xd.max(axis=1, keepdims=True)
    lse = (mx + np.log(np.exp(xd - mx).sum(axis=1, keepdims=True)))[:, 0]
    valid = labels != -100
    want_loss = np.where(valid, lse - xd[np.arange(rows), np.where(valid, labels, 0)], 0.0)
    np.testing.assert_allclose(loss, want_loss, rtol=1e-6, atol=1e-6)
    probs = np.exp(xd - lse[:, None])
    probs[np.arange(rows)[valid], labels[valid]] -= 1.0
    probs[~valid] = 0.0
    want_bits = oracle.bf16_rne(probs.astype(np.float32)).reshape(rows, vocab)
    diff = np.abs(grad_bits.astype(np.int32) - want_bits.astype(np.int32))
    # ulp distance on same-sign values; sign flips can only occur at |value| ~ 0
    assert diff.max() <= 1, (diff.max(), np.argwhere(diff > 1)[:4])
    assert (diff == 0).mean() > 0.99
    assert np.all(grad_bits[~valid] == 0)


def test_ce_rows_beyond_one_launch():
    """More rows than one launch of 1024-thread blocks holds (2^32 work-items): the
    entry point splits them, and every row still matches an fp64 restatement (here in
    torch float64 on the device, over all 4.2M rows)."""
    from torchure_amd import _native

    rows, v = 0xFFFFFFFF // 1024 + 2001, 16
    g = torch.Generator(device=DEV).manual_seed(11)
    # unit-scale logits: no row has a softmax entry within 1e-4 of 1, where fp32's
    # p - 1 cancels (the reference's fp32 softmax loses the same bits there)
    logits = torch.randn(rows, v, device=DEV, generator=g).to(torch.bfloat16)
    labels = torch.randint(0, v, (rows,), device=DEV, generator=g)
    labels[::1009] = -100
    xd = logits.double()
    work = logits.clone()
    loss = torch.empty(rows, dtype=torch.float32, device=DEV)
    rc = _native.lib().tm_ce_rows_bf16(work.data_ptr(), v, labels.data_ptr(), rows, v, -100,
                                       loss.data_ptr(), _native.stream_handle(DEV))
    _native.check(rc, "tm_ce_rows_bf16")
    valid = labels != -100
    lse = torch.logsumexp(xd, dim=1)
    picked = xd.gather(1, labels.clamp(min=0)[:, None])[:, 0]
    want = torch.where(valid, lse - picked, torch.zeros_like(lse))
    torch.testing.assert_close(loss.double(), want, rtol=1e-6, atol=1e-6)
    probs = torch.exp(xd - lse[:, None])
    probs[valid.nonzero()[:, 0], labels[valid]] -= 1.0
    probs[~valid] = 0.0
    want_bits = probs.float().to(torch.bfloat16).view(torch.int16).int()
    diff = (work.view(torch.int16).int() - want_bits).abs()
    assert int(diff.max()) <= 1
    assert float((diff == 0).double().mean()) > 0.99
    del xd, probs


@pytest.mark.parametrize("chunk", [None, 300])
def test_fused_linear_ce_matches_reference_composition(chunk):
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(7)
    n, d, v = 1000, 256, 4096
    hidden = (torch.randn(n, d, device=DEV, generator=g) * 1.0).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::37] = -100
    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    loss = fused_linear_cross_entropy(h1, w1, labels, -100, chunk)
    loss.backward()
    ref_loss, ref_gh, ref_gw = fused_linear_ce_reference(hidden, weight, labels, -100,
                                                         chunk_size=chunk or 1024)
    torch.cuda.synchronize()
    assert abs(loss.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
    gh_err = (h1.grad.float() - ref_gh.float()).abs().max().item()
    gw_err = (w1.grad - ref_gw).abs().max().item()
    print(f"chunk {chunk}: loss {loss.item():.6f} ref {ref_loss.item():.6f}, "
          f"max |d grad_h| {gh_err:.3e} (scale {ref_gh.float().abs().max().item():.3e}), "
          f"max |d grad_w| {gw_err:.3e} (scale {ref_gw.abs().max().item():.3e})")
    assert gh_err <= 1e-2 * ref_gh.float().abs().max().item()
    assert gw_err <= 1e-2 * ref_gw.abs().max().item()
    assert w1.grad.dtype == torch.float32 and h1.grad.dtype == torch.bfloat16


def test_fused_linear_ce_all_ignored_and_double_backward():
    from torchure_amd.loss import fused_linear_cross_entropy

    n, d, v = 64, 32, 512
    hidden = torch.randn(n, d, device=DEV).to(torch.bfloat16).requires_grad_(True)
    weight = (torch.randn(v, d, device=DEV) * 0.1).requires_grad_(True)
    labels = torch.full((n,), -100, dtype=torch.int64, device=DEV)
    loss = fused_linear_cross_entropy(hidden, weight, labels)
    loss.backward(retain_graph=True)
    assert loss.item() == 0.0
    assert torch.count_nonzero(hidden.grad).item() == 0 and torch.count_nonzero(weight.grad).item() == 0
    with pytest.raises(RuntimeError, match="backward called twice"):
        loss.backward()


@pytest.mark.parametrize("accumulate,scaled,n,offset", [
    (0, 0, 4096, 0), (1, 0, 4096, 0), (0, 1, 4096, 0), (1, 1, 4096, 0),
    (1, 1, 1003, 0), (1, 1, 2050, 1), (0, 1, 777, 3)])
def test_ce_grad_w_handover_bit_exact(accumulate, scaled, n, offset):
    """tm_ce_grad_w vs the reference's torch ops on the same data
    (fused_linear_ce.py:80-81 `grad_weight += gw` on a zero-filled fp32 buffer, :126
    `grad_weight.mul_(grad_out / n_valid)`), bit for bit, including -0, +-inf, NaN and
    subnormal bf16 inputs, odd sizes and buffers that are not 16-byte aligned."""
    from torchure_amd import _native

    r = H.rng(n + 7 * offset + accumulate)
    chunk_bits = oracle.bf16_rne((r.standard_normal(n + offset) * 0.3).astype(np.float32))
    chunk_bits[offset:offset + 6] = [0x8000, 0x0000, 0x7F80, 0xFF80, 0x7FC0, 0x0001]
    chunk = torch.from_numpy(chunk_bits.view(np.int16).copy()).to(DEV)[offset:]
    acc0 = torch.from_numpy((r.standard_normal(n + offset) * 0.1).astype(np.float32)).to(DEV)[offset:]
    acc0[0] = acc0[6] = -0.0  # -0 + -0 keeps the sign only when accumulating
    grad_out = torch.tensor([0.37], dtype=torch.float32, device=DEV)
    n_valid = torch.tensor([977.0], dtype=torch.float32, device=DEV)

    if accumulate:
        want = acc0.clone()
    else:
        want = torch.zeros(n, dtype=torch.float32, device=DEV)
    want += chunk.view(torch.bfloat16).float()
    if scaled:
        want.mul_(grad_out[0] / n_valid[0])

    got = acc0.clone() if accumulate else torch.full((n,), 123.0, device=DEV)
    got_base = torch.empty(n + offset, dtype=torch.float32, device=DEV)
    got_view = got_base[offset:]
    got_view.copy_(got)
    rc = _native.lib().tm_ce_grad_w(got_view.data_ptr(), chunk.data_ptr(), n, accumulate,
                                    grad_out.data_ptr() if scaled else None,
                                    n_valid.data_ptr() if scaled else None, _native.stream_handle(DEV))
    _native.check(rc, "tm_ce_grad_w")
    torch.cuda.synchronize()
    a = got_view.cpu().numpy().view(np.uint32)
    b = want.cpu().numpy().view(np.uint32)
    assert np.array_equal(a, b), np.argwhere(a != b)[:5]


@pytest.mark.parametrize("accumulate,scaled,n,offset", [
    (0, 0, 4096, 0), (1, 0, 4096, 0), (0, 1, 4096, 0), (1, 1, 4096, 0), (1, 1, 1003, 0), (0, 1, 777, 3)])
def test_ce_grad_w2_handover_bit_exact(accumulate, scaled, n, offset):
    """tm_ce_grad_w2 (two chunks in one pass) vs the reference's torch ops on the same data:
    `grad_weight += gw` for one chunk and then the next, on a zero-filled (or given) fp32
    buffer, then `mul_(grad_out / n_valid)` (fused_linear_ce.py:80-81,126), bit for bit,
    with -0, +-inf, NaN and subnormal bf16 inputs, odd sizes and unaligned buffers."""
    from torchure_amd import _native

    r = H.rng(3 * n + 11 * offset + accumulate + 5)
    bits = []
    for k in range(2):
        b = oracle.bf16_rne((r.standard_normal(n + offset) * 0.3).astype(np.float32))
        b[offset + 3 * k:offset + 3 * k + 6] = [0x8000, 0x0000, 0x7F80, 0xFF80, 0x7FC0, 0x0001]
        bits.append(torch.from_numpy(b.view(np.int16).copy()).to(DEV)[offset:])
    acc0 = torch.from_numpy((r.standard_normal(n + offset) * 0.1).astype(np.float32)).to(DEV)[offset:]
    acc0[0] = acc0[9] = -0.0
    grad_out = torch.tensor([0.37], dtype=torch.float32, device=DEV)
    n_valid = torch.tensor([977.0], dtype=torch.float32, device=DEV)

    want = acc0.clone() if accumulate else torch.zeros(n, dtype=torch.float32, device=DEV)
    want += bits[0].view(torch.bfloat16).float()
    want += bits[1].view(torch.bfloat16).float()
    if scaled:
        want.mul_(grad_out[0] / n_valid[0])

    got_base = torch.full((n + offset,), 123.0, dtype=torch.float32, device=DEV)
    got = got_base[offset:]
    if accumulate:
        got.copy_(acc0)
    rc = _native.lib().tm_ce_grad_w2(got.data_ptr(), bits[0].data_ptr(), bits[1].data_ptr(), n, accumulate,
                                     grad_out.data_ptr() if scaled else None,
                                     n_valid.data_ptr() if scaled else None, _native.stream_handle(DEV))
    _native.check(rc, "tm_ce_grad_w2")
    torch.cuda.synchronize()
    a = got.cpu().numpy().view(np.uint32)
    b = want.cpu().numpy().view(np.uint32)
    assert np.array_equal(a, b), np.argwhere(a != b)[:5]


@pytest.mark.parametrize("k,accumulate,scaled,n,offset", [
    (1, 0, 1, 4096, 0), (3, 1, 0, 4096, 0), (5, 0, 0, 1003, 0), (8, 1, 1, 4096, 0),
    (8, 0, 1, 2050, 1), (7, 1, 1, 777, 3)])
def test_ce_grad_w_fold_bit_exact(k, accumulate, scaled, n, offset):
    """tm_ce_grad_w_fold (k chunks in one pass) vs the reference's torch ops on the same data:
    `grad_weight += gw` once per chunk in order, on a zero-filled (or given) fp32 buffer, then
    `mul_(grad_out / n_valid)` (fused_linear_ce.py:80-81,126), bit for bit, with -0, +-inf, NaN
    and subnormal bf16 inputs, odd sizes and buffers that are not 16-byte aligned."""
    import ctypes

    from torchure_amd import _native

    r = H.rng(5 * n + 13 * offset + 17 * k + accumulate)
    bits = []
    for j in range(k):
        b = oracle.bf16_rne((r.standard_normal(n + offset) * 0.3).astype(np.float32))
        b[offset + 2 * j:offset + 2 * j + 6] = [0x8000, 0x0000, 0x7F80, 0xFF80, 0x7FC0, 0x0001]
        bits.append(torch.from_numpy(b.view(np.int16).copy()).to(DEV)[offset:])
    acc0 = torch.from_numpy((r.standard_normal(n + offset) * 0.1).astype(np.float32)).to(DEV)[offset:]
    acc0[0] = acc0[20] = -0.0
    grad_out = torch.tensor([0.37], dtype=torch.float32, device=DEV)
    n_valid = torch.tensor([977.0], dtype=torch.float32, device=DEV)

    want = acc0.clone() if accumulate else torch.zeros(n, dtype=torch.float32, device=DEV)
    for b in bits:
        want += b.view(torch.bfloat16).float()
    if scaled:
        want.mul_(grad_out[0] / n_valid[0])

    got_base = torch.full((n + offset,), 123.0, dtype=torch.float32, device=DEV)
    got = got_base[offset:]
    if accumulate:
        got.copy_(acc0)
    ptrs = (ctypes.c_void_p * k)(*[b.data_ptr() for b in bits])
    rc = _native.lib().tm_ce_grad_w_fold(got.data_ptr(), ptrs, k, n, accumulate,
                                         grad_out.data_ptr() if scaled else None,
                                         n_valid.data_ptr() if scaled else None, _native.stream_handle(DEV))
    _native.check(rc, "tm_ce_grad_w_fold")
    torch.cuda.synchronize()
    a = got.cpu().numpy().view(np.uint32)
    w = want.cpu().numpy().view(np.uint32)
    assert np.array_equal(a, w), np.argwhere(a != w)[:5]


@pytest.mark.parametrize("chunk", [700, 350, 256, 175, 128, 100, 80, 64, 40])
def test_fused_linear_ce_grad_w_equals_chunkwise_reference_ops(chunk):
    """Folding the chunks' hand-overs and deferring the last chunk change nothing: grad_W of
    the op with 1, 2, 3, 4, 7, 9 and 18 chunks (folds of 8 in forward, the rest with the last
    in backward) equals, bit for bit, the reference's chunk loop run
    on the same kernels -- zero buffer, `+=` of each chunk's bf16 grad_W, then
    `mul_(grad_out / n_valid)` (fused_linear_ce.py:67-91,117-126) -- and grad_h likewise
    (`grad_hidden[s:e] = gh`, then `mul_(scale.to(bf16))`)."""
    from torchure_amd import _native
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(11)
    n, d, v = 700, 128, 2048
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::13] = -100
    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    loss = fused_linear_cross_entropy(h1, w1, labels, -100, chunk)
    (loss * 3.0).backward()
    gh_ref, gw_ref = _chunk_loop_on_the_same_kernels(hidden, weight, labels, chunk, 3.0)
    torch.cuda.synchronize()
    assert torch.equal(w1.grad.view(torch.int32), gw_ref.view(torch.int32))
    assert torch.equal(h1.grad.view(torch.int16), gh_ref.view(torch.int16))


def _chunk_loop_on_the_same_kernels(hidden, weight, labels, chunk, grad_out):
    """The reference's chunk loop (fused_linear_ce.py:67-91,117-126) run on this build's GEMMs
    and row kernel: a zero fp32 grad_W, `+=` of each chunk's bf16 grad_W, `grad_hidden[s:e] =
    gh`, then both scaled by grad_out / n_valid (grad_h by its bf16 rounding)."""
    from torchure_amd import _native
    from torchure_amd.loss.fused_linear_ce import GradHidden, _grad_w, _logits

    n, v = hidden.shape[0], weight.shape[0]
    lib = _native.lib()
    stream = _native.stream_handle(DEV)
    w = weight.to(torch.bfloat16).contiguous()
    gw_ref = torch.zeros(weight.shape, dtype=torch.float32, device=DEV)
    gh_ref = torch.empty_like(hidden)
    row_loss = torch.empty(n, dtype=torch.float32, device=DEV)
    grad_h = GradHidden(w, [min(chunk, n - s) for s in range(0, n, chunk)], lib, stream)
    for s in range(0, n, chunk):
        e = min(s + chunk, n)
        logits = _logits(hidden[s:e], w, lib, stream)
        _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v, -100,
                                          row_loss[s:].data_ptr(), stream), "tm_ce_rows_bf16")
        gh = torch.empty((e - s, w.shape[1]), dtype=torch.bfloat16, device=DEV)
        grad_h(logits, gh)
        gh_ref[s:e] = gh
        gw_ref += _grad_w(logits, hidden[s:e], lib, stream)
    n_valid = (labels != -100).sum().clamp_min(1)
    scale = torch.tensor(grad_out, device=DEV) / n_valid
    gw_ref.mul_(scale)
    gh_ref.mul_(scale.to(torch.bfloat16))
    return gh_ref, gw_ref


def test_default_chunking_is_the_reference_1024_rows():
    """Called without chunk_size, the op chunks by 1024 rows, the reference's default
    (fused_linear_ce.py:131): grad_W and grad_h equal the reference's chunk loop at 1024 rows
    bit for bit (2600 rows: chunks of 1024, 1024 and 552). chunk_size=None and "auto" take the
    4 GiB logits budget instead, here one chunk: the bits of chunk_size=2600."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(12)
    n, d, v = 2600, 128, 2048
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::17] = -100

    def run(*chunk_arg):
        h = hidden.clone().requires_grad_(True)
        w = weight.clone().requires_grad_(True)
        fused_linear_cross_entropy(h, w, labels, -100, *chunk_arg).backward()
        return h.grad, w.grad

    gh, gw = run()
    gh_ref, gw_ref = _chunk_loop_on_the_same_kernels(hidden, weight, labels, 1024, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(gw.view(torch.int32), gw_ref.view(torch.int32))
    assert torch.equal(gh.view(torch.int16), gh_ref.view(torch.int16))
    gh_one, gw_one = run(n)
    for auto in (None, "auto"):
        gh_a, gw_a = run(auto)
        assert torch.equal(gw_a.view(torch.int32), gw_one.view(torch.int32))
        assert torch.equal(gh_a.view(torch.int16), gh_one.view(torch.int16))
    with pytest.raises(ValueError, match="chunk_size"):
        run("large")


def test_out_of_range_label_gives_nan_loss():
    """A label outside [0, vocab) other than ignore_index is an error in the reference (its
    gather asserts on the device); here the row loss, and so the mean loss, is NaN."""
    labels = np.array([3, -1, 100000, -100, 7], dtype=np.int64)
    r = H.rng(11)
    bits = oracle.bf16_rne((r.standard_normal((5, 4096)) * 2.0).astype(np.float32)).reshape(5, 4096)
    _, loss = _ce_rows(bits, labels, -100)
    assert np.isfinite(loss[[0, 4]]).all() and loss[3] == 0.0
    assert np.isnan(loss[1]) and np.isnan(loss[2])


@pytest.mark.parametrize("v", [4096, 1001, 200000])
def test_ce_rows_edge_rows_vs_fp64(v):
    """Rows the random tests do not reach: masked vocabulary entries (-inf), a range wide
    enough that most results are denormal or zero (the full-range exp fallback), constant
    rows, large magnitudes, and a label on a -inf logit (infinite loss). On the in-register
    path (4096), the element-wise path (1001: rows not 16-byte aligned) and the two-read
    path (200000)."""
    r = H.rng(21)
    rows = []
    x = (r.standard_normal(v) * 2.0).astype(np.float32); x[::3] = -np.inf; rows.append(x)      # masked
    x = np.linspace(-200.0, 20.0, v).astype(np.float32); rows.append(x)                       # denormal tail
    rows.append(np.full(v, 1.5, dtype=np.float32))                                            # constant
    x = (r.standard_normal(v) * 1e4).astype(np.float32); rows.append(x)                       # large spread
    x = (r.standard_normal(v) + 1e30).astype(np.float32); rows.append(x)                      # huge offset
    x = (r.standard_normal(v)).astype(np.float32); x[5] = -np.inf; rows.append(x)             # label on -inf
    bits = oracle.bf16_rne(np.stack(rows)).reshape(len(rows), v)
    labels = np.array([1, v - 96, 7, 123, 99, 5], dtype=np.int64)
    grad_bits, loss = _ce_rows(bits, labels, -100)
    xd = oracle.bf16_to_f32(bits).reshape(len(rows), v).astype(np.float64)
    mx = xd.max(axis=1, keepdims=True)
    lse = (mx + np.log(np.exp(xd - mx).sum(axis=1, keepdims=True)))[:, 0]
    want_loss = lse - xd[np.arange(len(rows)), labels]
    assert np.isinf(loss[5]) and loss[5] > 0
    np.testing.assert_allclose(loss[:5], want_loss[:5], rtol=1e-6, atol=1e-6)
    probs = np.exp(xd - lse[:, None])
    probs[np.arange(len(rows)), labels] -= 1.0
    want_bits = oracle.bf16_rne(probs.astype(np.float32)).reshape(len(rows), v)
    diff = np.abs(grad_bits.astype(np.int32) - want_bits.astype(np.int32))
    assert diff.max() <= 1, (diff.max(), np.argwhere(diff > 1)[:4])
    assert np.all(grad_bits[0, ::3] == 0)  # exp(-inf) = 0 exactly


@pytest.mark.parametrize("b,s,d,v,chunk,ignore_frac,hidden_dtype", [
    (2, 128, 64, 1000, 64, 0.1, torch.bfloat16),          # uneven chunks
    (2, 256, 128, 5000, 512, 0.0, torch.bfloat16),        # one chunk
    (2, 4096, 1024, 151936, 1024, 0.05, torch.bfloat16),  # the Qwen3 head at the reference's chunk size
    (2, 4096, 1024, 151936, None, 0.05, torch.bfloat16),  # the same with this build's default (one chunk)
    (2, 4096, 1024, 151936, 4096, 0.05, torch.float32),   # the trainer's call: fp32 hidden, autocast
])
def test_reference_cases_vs_plain_cross_entropy(b, s, d, v, chunk, ignore_frac, hidden_dtype):
    """The cases and bars of the reference's own test (tests/fused_linear_ce.py:23-56): the
    op against an unfused lm_head + F.cross_entropy on fp32 logits, through autograd, with
    bf16 hidden states and an fp32 head weight: |loss difference| < 2e-3 * max(1, loss) and
    relative L2 error of both grads < 3e-2. The unfused side uses 2-D products only. The
    last case is the trainer's own call (objectives/autoregressive.py:38-44, ce_chunk_size 4096 from :21):
    fp32 hidden states with both sides run under bf16 autocast."""
    import contextlib

    import torch.nn.functional as F

    from torchure_amd.loss import fused_linear_cross_entropy

    fp32 = hidden_dtype == torch.float32
    amp = (lambda: torch.autocast("cuda", dtype=torch.bfloat16)) if fp32 else contextlib.nullcontext
    torch.manual_seed(0)
    hidden = (torch.randn(b, s, d, device=DEV, dtype=torch.bfloat16) * 0.5).to(hidden_dtype)
    weight = torch.randn(v, d, device=DEV, dtype=torch.float32) * 0.02
    labels = torch.randint(0, v, (b, s), device=DEV)
    labels[torch.rand(b, s, device=DEV) < ignore_frac] = -100

    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    with amp():
        logits = h1.reshape(-1, d) @ w1.to(torch.bfloat16).t()
        loss_ref = F.cross_entropy(logits.float(), labels.reshape(-1), ignore_index=-100)
    loss_ref.backward()
    del logits

    h2 = hidden.clone().requires_grad_(True)
    w2 = weight.clone().requires_grad_(True)
    with amp():
        loss = fused_linear_cross_entropy(h2, w2, labels, -100, chunk)
    loss.backward()

    def rel(a, b_):
        return float((a.float() - b_.float()).norm() / b_.float().norm().clamp_min(1e-12))

    dh, dw = rel(h2.grad, h1.grad), rel(w2.grad, w1.grad)
    print(f"V={v} chunk={chunk}: loss {loss.item():.6f} vs {loss_ref.item():.6f}, rel dh {dh:.2e}, dw {dw:.2e}")
    assert abs(loss_ref.item() - loss.item()) < 2e-3 * max(1.0, loss_ref.item())
    assert dh < 3e-2
    assert dw < 3e-2
    assert h2.grad.dtype == hidden_dtype and h1.grad.dtype == hidden_dtype and w2.grad.dtype == torch.float32


@pytest.mark.parametrize("vocab", [4096, 1001, 200000])
def test_loss_only_rows_equal_gradient_rows(vocab):
    """tm_ce_rows_loss_bf16 gives the row losses of tm_ce_rows_bf16 bit for bit (register,
    element-wise and streaming paths) and leaves the logits untouched."""
    from torchure_amd import _native

    g = torch.Generator(device=DEV).manual_seed(vocab)
    rows = 29
    logits = (torch.randn(rows, vocab, device=DEV, generator=g) * 3.0).to(torch.bfloat16)
    labels = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
    labels[[2, 11]] = -100
    keep = logits.clone()
    a = torch.empty(rows, device=DEV)
    b = torch.empty(rows, device=DEV)
    lib, s = _native.lib(), _native.stream_handle(DEV)
    _native.check(lib.tm_ce_rows_loss_bf16(logits.data_ptr(), vocab, labels.data_ptr(), rows, vocab, -100,
                                           a.data_ptr(), s), "tm_ce_rows_loss_bf16")
    assert torch.equal(logits.view(torch.int16), keep.view(torch.int16))
    _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), vocab, labels.data_ptr(), rows, vocab, -100,
                                      b.data_ptr(), s), "tm_ce_rows_bf16")
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("chunk", [None, 300])
def test_loss_without_grad_and_partial_grads(chunk):
    """Under torch.no_grad the op takes the loss-only path and returns the training path's
    loss bit for bit. With only the weight (or only the hidden states) requiring a
    gradient, that gradient equals the one computed with both, bit for bit, and the other
    input gets none."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(3)
    n, d, v = 1000, 256, 4096
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::23] = -100

    h = hidden.clone().requires_grad_(True)
    w = weight.clone().requires_grad_(True)
    loss = fused_linear_cross_entropy(h, w, labels, -100, chunk)
    loss.backward()
    with torch.no_grad():
        eval_loss = fused_linear_cross_entropy(h, w, labels, -100, chunk)
    assert not eval_loss.requires_grad
    assert eval_loss.view(torch.int32).item() == loss.detach().view(torch.int32).item()
    # inputs that require no gradient: the loss-only path too
    plain = fused_linear_cross_entropy(hidden, weight, labels, -100, chunk)
    assert plain.view(torch.int32).item() == loss.detach().view(torch.int32).item()

    w_only = weight.clone().requires_grad_(True)
    l1 = fused_linear_cross_entropy(hidden, w_only, labels, -100, chunk)
    l1.backward()
    assert torch.equal(w_only.grad, w.grad)
    assert l1.detach().view(torch.int32).item() == loss.detach().view(torch.int32).item()

    h_only = hidden.clone().requires_grad_(True)
    l2 = fused_linear_cross_entropy(h_only, weight, labels, -100, chunk)
    l2.backward()
    assert torch.equal(h_only.grad.view(torch.int16), h.grad.view(torch.int16))


@pytest.mark.parametrize("chunk", [None, 300])
def test_fp32_hidden_under_autocast(chunk):
    """fp32 hidden states inside bf16 autocast, the reference trainer's call: the products
    run on autocast's bf16 casts and grad_hidden is fp32 = float(bf16 GEMM result) * scale
    (fused_linear_ce.py:68,80,120). With 512 valid rows the scale is a power of two, so both
    scalings are exact and the fp32 path's results follow bit for bit from the bf16 path's on
    hidden.to(bf16): the same loss, the same grad_W, and grad_h widened exactly. Against the
    reference composition run under autocast the bars of the composition test hold, and fp16
    autocast is refused."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(11)
    n, d, v = 1000, 256, 4096
    hidden = torch.randn(n, d, device=DEV, generator=g)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[torch.randperm(n, device=DEV, generator=g)[:n - 512]] = -100

    hb = hidden.to(torch.bfloat16).requires_grad_(True)
    wb = weight.clone().requires_grad_(True)
    loss_b = fused_linear_cross_entropy(hb, wb, labels, -100, chunk)
    loss_b.backward()

    hf = hidden.clone().requires_grad_(True)
    wf = weight.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss_f = fused_linear_cross_entropy(hf, wf, labels, -100, chunk)
    loss_f.backward()
    assert hf.grad.dtype == torch.float32 and wf.grad.dtype == torch.float32
    assert loss_f.dtype == torch.float32
    assert loss_f.detach().view(torch.int32).item() == loss_b.detach().view(torch.int32).item()
    assert torch.equal(wf.grad.view(torch.int32), wb.grad.view(torch.int32))
    assert torch.equal(hf.grad.view(torch.int32), hb.grad.float().view(torch.int32))

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        eval_loss = fused_linear_cross_entropy(hidden, weight, labels, -100, chunk)
    assert eval_loss.view(torch.int32).item() == loss_b.detach().view(torch.int32).item()

    # a scale that is not a power of two, against the reference composition under autocast
    labels2 = labels.clone()
    labels2[::37] = -100
    h2 = hidden.clone().requires_grad_(True)
    w2 = weight.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss2 = fused_linear_cross_entropy(h2, w2, labels2, -100, chunk)
        ref_loss, ref_gh, ref_gw = fused_linear_ce_reference(hidden, weight, labels2, -100,
                                                             chunk_size=chunk or 1024)
    loss2.backward()
    torch.cuda.synchronize()
    assert ref_gh.dtype == torch.float32
    assert abs(loss2.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
    gh_err = (h2.grad - ref_gh).abs().max().item()
    gw_err = (w2.grad - ref_gw).abs().max().item()
    print(f"fp32 hidden, chunk {chunk}: loss {loss2.item():.6f} ref {ref_loss.item():.6f}, "
          f"max |d grad_h| {gh_err:.3e}, max |d grad_w| {gw_err:.3e}")
    assert gh_err <= 1e-2 * ref_gh.abs().max().item()
    assert gw_err <= 1e-2 * ref_gw.abs().max().item()

    with pytest.raises(NotImplementedError, match="autocast"), torch.autocast("cuda", dtype=torch.float16):
        fused_linear_cross_entropy(hidden, weight, labels)
    # bf16 hidden under fp16 autocast: autocast would make the logits fp16, so it is refused too
    with pytest.raises(NotImplementedError, match="autocast"), torch.autocast("cuda", dtype=torch.float16):
        fused_linear_cross_entropy(hidden.to(torch.bfloat16).requires_grad_(True), weight, labels)
    with pytest.raises(NotImplementedError, match="autocast"), torch.autocast("cuda", dtype=torch.float16):
        with torch.no_grad():
            fused_linear_cross_entropy(hidden.to(torch.bfloat16), weight, labels)


@pytest.mark.parametrize("ignore_index", [7, 0])
def test_ignore_index_inside_the_vocabulary(ignore_index):
    """ignore_index may be a real class id (F.cross_entropy semantics, fused_linear_ce.py:40,86):
    rows labelled with it are left out of the loss, the mean and both gradients, and the class
    is still scored for the other rows. Checked against the reference composition with the same
    ignore_index, in one chunk and in several, at that test's bars."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(100 + ignore_index)
    n, d, v = 700, 128, 1000
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[labels == ignore_index] = (ignore_index + 2) % v  # only the rows set below are ignored
    labels[1::9] = (ignore_index + 1) % v  # the neighbouring class, scored as usual
    labels[::5] = ignore_index
    for chunk in (None, 128):
        h = hidden.clone().requires_grad_(True)
        w = weight.clone().requires_grad_(True)
        loss = fused_linear_cross_entropy(h, w, labels, ignore_index, chunk)
        loss.backward()
        ref_loss, ref_gh, ref_gw = fused_linear_ce_reference(hidden, weight, labels, ignore_index,
                                                             chunk_size=chunk or 1024)
        torch.cuda.synchronize()
        assert abs(loss.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
        assert (h.grad[::5] == 0).all()  # ignored rows get no gradient
        assert (h.grad[1::5].abs().sum(dim=1) > 0).all()
        gh_err = (h.grad.float() - ref_gh.float()).abs().max().item()
        gw_err = (w.grad - ref_gw).abs().max().item()
        assert gh_err <= 1e-2 * ref_gh.float().abs().max().item()
        assert gw_err <= 1e-2 * ref_gw.abs().max().item()
        with torch.no_grad():
            ev = fused_linear_cross_entropy(hidden, weight, labels, ignore_index, chunk)
        assert ev.view(torch.int32).item() == loss.detach().view(torch.int32).item()


def test_non_contiguous_inputs_give_the_contiguous_bits():
    """hidden as a transposed view and a strided weight slice: the op works on contiguous
    copies (as torch's products accept any strides), so loss and both gradients equal the
    contiguous call bit for bit, and the gradients reach the views' bases."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(21)
    n, d, v = 600, 128, 3000
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::11] = -100

    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    l1 = fused_linear_cross_entropy(h1, w1, labels, -100, 256)
    l1.backward()

    hbase = hidden.t().contiguous().requires_grad_(True)  # (d, n); its transpose is (n, d), strided
    wbase = torch.zeros(v, 2 * d, device=DEV)
    wbase[:, ::2] = weight
    wbase.requires_grad_(True)
    h2, w2 = hbase.t(), wbase[:, ::2]
    assert not h2.is_contiguous() and not w2.is_contiguous()
    l2 = fused_linear_cross_entropy(h2, w2, labels, -100, 256)
    l2.backward()
    torch.cuda.synchronize()
    assert l1.detach().view(torch.int32).item() == l2.detach().view(torch.int32).item()
    assert torch.equal(hbase.grad.t().contiguous().view(torch.int16), h1.grad.view(torch.int16))
    assert torch.equal(wbase.grad[:, ::2].contiguous().view(torch.int32), w1.grad.view(torch.int32))
    assert torch.count_nonzero(wbase.grad[:, 1::2]).item() == 0


@pytest.mark.parametrize("vocab", [4096, 1001, 151936])
def test_ce_rows_f32_kernel_vs_fp64(vocab):
    """tm_ce_rows_f32 (fp32 logits, the fp32-hidden path outside autocast) against an fp64
    restatement of fused_linear_ce.py:39-51 on the same fp32 logits: row losses within 1e-6
    relative; gradients within 2e-6 relative of exp(x - lse), plus the fp32 rounding of lse and
    of x - lse (2^-23 of their magnitudes), plus 1e-7 absolute at the label (p - 1 cancels);
    ignored rows exactly zero; tm_ce_rows_loss_f32 gives the same loss bits
    and leaves the logits untouched. V = 1001 takes the element-wise path (rows not 16-byte
    aligned), and rows hold -inf entries and a wide range."""
    from torchure_amd import _native

    g = torch.Generator(device=DEV).manual_seed(vocab)
    rows = 64
    x = torch.randn(rows, vocab, device=DEV, generator=g) * 4.0
    x[3, ::7] = float("-inf")
    x[5] *= 20.0
    labels = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
    labels[::9] = -100
    labels[3] = 1  # a finite entry of the masked row
    lib, stream = _native.lib(), _native.stream_handle(DEV)
    work = x.clone()
    loss = torch.empty(rows, dtype=torch.float32, device=DEV)
    _native.check(lib.tm_ce_rows_f32(work.data_ptr(), vocab, labels.data_ptr(), rows, vocab, -100,
                                     loss.data_ptr(), stream), "tm_ce_rows_f32")
    ro = x.clone()
    loss2 = torch.empty(rows, dtype=torch.float32, device=DEV)
    _native.check(lib.tm_ce_rows_loss_f32(ro.data_ptr(), vocab, labels.data_ptr(), rows, vocab, -100,
                                          loss2.data_ptr(), stream), "tm_ce_rows_loss_f32")
    xd = x.double()
    lse = torch.logsumexp(xd, dim=1)
    valid = labels != -100
    picked = xd.gather(1, labels.clamp(min=0)[:, None])[:, 0]
    want_loss = torch.where(valid, lse - picked, torch.zeros_like(lse))
    p = torch.exp(xd - lse[:, None])
    want = p.clone()
    idx = valid.nonzero()[:, 0]
    want[idx, labels[idx]] -= 1.0
    want[~valid] = 0.0
    torch.cuda.synchronize()
    assert torch.equal(ro, x)
    assert torch.equal(loss.view(torch.int32), loss2.view(torch.int32))
    torch.testing.assert_close(loss.double(), want_loss, rtol=1e-6, atol=1e-6)
    err = (work.double() - want).abs()
    # fp32 rounding of lse (half an ulp of |lse|) and of the difference x - lse move the
    # exponent by up to (|lse| + |x - lse|) * 2^-24 each
    dist = (xd - lse[:, None]).abs()
    dist = torch.where(torch.isfinite(dist), dist, torch.zeros_like(dist))  # -inf entries: p = 0 exactly
    rel = 2e-6 + (lse.abs()[:, None] + dist) * 2.0 ** -23
    bound = p * rel + 1e-7 * (want != p).double() + 1e-30
    bound[~valid] = 0.0
    assert bool((err <= bound).all()), float((err / bound.clamp_min(1e-300)).max())
    assert bool((work[~valid] == 0).all())


@pytest.mark.parametrize("chunk", [None, 300])
def test_fp32_hidden_without_autocast(chunk):
    """fp32 hidden states outside autocast: the reference runs fp32 GEMMs on w =
    weight.to(fp32) (fused_linear_ce.py:38,52,57,65) and returns fp32 gradients. Against the
    reference composition (the same torch calls) on the same device: loss within 1e-6
    relative, both gradients within 1e-5 of their scale; against an fp64 unfused cross
    entropy: loss within 1e-5 relative and gradients within 1e-4 relative L2. The loss-only
    call gives the training loss bits; a bf16 weight gets its gradient as autograd hands it
    over (fp32 cast to the weight's dtype), as in the reference."""
    import torch.nn.functional as F

    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(23)
    n, d, v = 1000, 256, 4096
    hidden = torch.randn(n, d, device=DEV, generator=g)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::37] = -100
    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    loss = fused_linear_cross_entropy(h1, w1, labels, -100, chunk)
    (loss * 2.0).backward()
    assert loss.dtype == torch.float32 and h1.grad.dtype == torch.float32 and w1.grad.dtype == torch.float32
    ref_loss, ref_gh, ref_gw = fused_linear_ce_reference(hidden, weight, labels, -100, chunk_size=chunk or n)
    torch.cuda.synchronize()
    assert abs(loss.item() - ref_loss.item()) <= 1e-6 * abs(ref_loss.item())
    assert (h1.grad - 2.0 * ref_gh).abs().max().item() <= 1e-5 * ref_gh.abs().max().item() * 2.0
    assert (w1.grad - 2.0 * ref_gw).abs().max().item() <= 1e-5 * ref_gw.abs().max().item() * 2.0

    hd = hidden.double().requires_grad_(True)
    wd = weight.double().requires_grad_(True)
    ld = F.cross_entropy(hd @ wd.t(), labels, ignore_index=-100)
    (ld * 2.0).backward()

    def rel(a, b):
        return float((a.double() - b).norm() / b.norm())

    assert abs(loss.item() - ld.item()) <= 1e-5 * ld.item()
    assert rel(h1.grad, hd.grad) < 1e-4 and rel(w1.grad, wd.grad) < 1e-4

    with torch.no_grad():
        ev = fused_linear_cross_entropy(hidden, weight, labels, -100, chunk)
    assert ev.view(torch.int32).item() == loss.detach().view(torch.int32).item()

    wb = weight.to(torch.bfloat16).requires_grad_(True)
    h2 = hidden.clone().requires_grad_(True)
    fused_linear_cross_entropy(h2, wb, labels, -100, chunk).backward()
    assert wb.grad.dtype == torch.bfloat16 and h2.grad.dtype == torch.float32
    with pytest.raises(NotImplementedError, match="float16"):
        fused_linear_cross_entropy(hidden.half().requires_grad_(True), weight, labels)


def test_fp32_weight_with_current_working_copy():
    """An fp32 head weight with an attached bf16 working copy: while the copy is current the op
    reads it instead of casting the master, with the cast's bits (loss, grad_h and grad_W equal a
    weight without a copy, bit for bit, training and loss-only); the copy really is what the op
    reads (bytes overwritten behind autograd's back change the loss, and a refresh restores it);
    a master modified in place makes the copy stale and the op casts again; after AdamW.step()
    the copy is current again, and a copy modified in place through torch is not taken."""
    import torchure_amd as ta
    from torchure_amd import _native
    from torchure_amd.loss import fused_linear_cross_entropy
    from torchure_amd.optimizer.working import current_copy

    g = torch.Generator(device=DEV).manual_seed(31)
    n, d, v = 1500, 256, 6000
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::9] = -100
    master = torch.nn.Parameter(torch.randn(v, d, device=DEV, generator=g) * 0.05)
    (copy,) = ta.attach_bf16_working_params([master])

    def run(weight):
        h = hidden.clone().requires_grad_(True)
        loss = fused_linear_cross_entropy(h, weight, labels, -100, 512)
        gh, gw = torch.autograd.grad(loss, (h, weight))
        with torch.no_grad():
            eval_loss = fused_linear_cross_entropy(hidden, weight, labels, -100, 512)
        return loss.detach(), gh, gw, eval_loss

    def same(a, b):
        return all(torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x.view(torch.int16),
                               y.view(torch.int32) if y.dtype == torch.float32 else y.view(torch.int16))
                   for x, y in zip(a, b))

    plain = torch.nn.Parameter(master.detach().clone())
    assert same(run(master), run(plain))
    assert torch.equal(run(master)[0], run(plain)[3])  # loss-only gives the training bits

    # overwrite the copy's bytes without an autograd version bump: the op reads the copy
    junk = (torch.randn(v, d, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    _native.check(_native.lib().tm_stream_copy(copy.data_ptr(), junk.data_ptr(), junk.numel() * 2,
                                               _native.stream_handle(DEV)), "tm_stream_copy")
    torch.cuda.synchronize()
    assert not torch.equal(run(master)[0], run(plain)[0])
    ta.refresh_bf16_working_params([master])
    assert same(run(master), run(plain))

    # a master changed in place: the copy is stale, the op casts the master again
    with torch.no_grad():
        master.mul_(1.5)
        plain.mul_(1.5)
    _native.check(_native.lib().tm_stream_copy(copy.data_ptr(), junk.data_ptr(), junk.numel() * 2,
                                               _native.stream_handle(DEV)), "tm_stream_copy")
    torch.cuda.synchronize()
    assert same(run(master), run(plain))
    # AdamW.step() writes the copy with the master, so the op reads it again afterwards
    ta.refresh_bf16_working_params([master])
    opt = ta.AdamW([master], lr=1e-3, fused=True)
    master.grad = torch.randn(v, d, device=DEV, generator=g) * 1e-3
    opt.step()
    with torch.no_grad():
        plain.copy_(master)
    assert current_copy(master) is copy
    assert same(run(master), run(plain))
    # a copy changed in place through torch is no longer taken for the cast
    with torch.no_grad():
        copy.add_(1.0)
    assert current_copy(master) is None
    assert same(run(master), run(plain))


def test_offset_working_copy_is_not_taken():
    """A current bf16 working copy that starts 2 bytes past a 16-byte boundary (the optimizer
    accepts copies at any offset) is not read by the op, whose kernels read the weight in
    16-byte vectors: the op casts the master instead and gives the bits of a weight without a
    copy, training and loss-only."""
    from torchure_amd.loss import fused_linear_cross_entropy
    from torchure_amd.loss.fused_linear_ce import _bf16_weight
    from torchure_amd.optimizer.working import current_copy, mark_current

    g = torch.Generator(device=DEV).manual_seed(37)
    n, d, v = 1024, 256, 4096
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    master = torch.nn.Parameter(torch.randn(v, d, device=DEV, generator=g) * 0.05)
    pool = torch.zeros(v * d + 8, dtype=torch.bfloat16, device=DEV)
    copy = pool[1:1 + v * d].view(v, d)
    assert copy.data_ptr() % 16 == 2
    copy.copy_(master.detach().to(torch.bfloat16))
    master._tm_working = copy
    mark_current(master, copy)
    assert current_copy(master) is copy
    assert _bf16_weight(master).data_ptr() % 16 == 0
    plain = torch.nn.Parameter(master.detach().clone())

    def run(weight):
        h = hidden.clone().requires_grad_(True)
        loss = fused_linear_cross_entropy(h, weight, labels, -100, 512)
        gh, gw = torch.autograd.grad(loss, (h, weight))
        with torch.no_grad():
            eval_loss = fused_linear_cross_entropy(hidden, weight, labels, -100, 512)
        return loss.detach(), gh, gw, eval_loss

    for x, y in zip(run(master), run(plain)):
        assert torch.equal(x, y)


def test_two_calls_on_two_streams_equal_sequential():
    """Two calls issued back to back from the host on two streams, with no synchronisation
    between them, give the bits of the same two calls run one after the other on one stream:
    each call's stream waits for the previous call's work on the device (CallOrder), so the
    two calls' GEMMs never run at the same time. The shapes use the Qwen3 head's width and the
    reference's 1024-row chunks."""
    from torchure_amd.loss import fused_linear_cross_entropy

    g = torch.Generator(device=DEV).manual_seed(41)
    n, d, v = 2048, 1024, 32768
    inputs = []
    for _ in range(2):
        hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
        weight = (torch.randn(v, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
        labels = torch.randint(0, v, (n,), device=DEV, generator=g)
        inputs.append((hidden, weight, labels))

    def one(hidden, weight, labels):
        h = hidden.clone().requires_grad_(True)
        w = weight.clone().requires_grad_(True)
        loss = fused_linear_cross_entropy(h, w, labels, -100, 1024)
        loss.backward()
        return loss.detach(), h.grad, w.grad

    torch.cuda.synchronize()
    seq = [one(*x) for x in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(DEV))
    out = []
    for s, x in zip(streams, inputs):
        with torch.cuda.stream(s):
            out.append(one(*x))
    torch.cuda.synchronize()
    for a, b in zip(seq, out):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
