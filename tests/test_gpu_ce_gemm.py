"""GPU parity of the split-K MFMA GEMM that computes the fused CE's grad_hidden
(tm_ce_grad_h_bf16: grad_h = grad_logits @ W, torchure/loss/fused_linear_ce.py:52) and of
the W^T it reads (tm_ce_transpose_bf16).

Checks:
- the transpose bit for bit against torch's;
- the GEMM against an fp64 product of the same bf16 operands: every element within one bf16
  ulp of the exact value plus 2^-20 of sum_k |a_ik b_kj| (the fp32 accumulation), at chunk
  shapes from one output tile with more splits than K slices up to the Qwen3 head's 1024 x
  151,936 x 1024 and a 4096-row chunk of a 2560-wide head;
- against torch.matmul (hipBLASLt) on the same operands: within one bf16 ulp plus the two
  fp32 accumulation budgets everywhere, and equal on at least 99% of the elements (the two
  differ only in fp32 summation order);
- deterministic: the same bits on a repeat call over a workspace holding other data;
- inside the op: the fused CE's grad_h on eligible chunks equals the GEMM's result for the
  chunk's grad_logits, and the whole op stays within the reference composition's bars.
"""

from __future__ import annotations

import pytest
import torch

from oracle.torch_composition import fused_linear_ce_reference

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import torchure_amd

    torchure_amd._native.lib()
    yield


def _lib():
    from torchure_amd import _native

    return _native, _native.lib(), _native.stream_handle(DEV)


def _transpose(w):
    native, lib, stream = _lib()
    v, d = w.shape
    wt = torch.empty((d, v), dtype=torch.bfloat16, device=DEV)
    native.check(lib.tm_ce_transpose_bf16(wt.data_ptr(), w.data_ptr(), v, d, stream), "tm_ce_transpose_bf16")
    return wt


def _grad_h(a, w, ws_fill=None):
    native, lib, stream = _lib()
    rows, vocab = a.shape
    dim = w.shape[1]
    wt = _transpose(w)
    nbytes = lib.tm_ce_grad_h_workspace_bytes(rows, vocab, dim)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    if ws_fill is not None:
        ws.fill_(ws_fill)
    out = torch.empty((rows, dim), dtype=torch.bfloat16, device=DEV)
    native.check(lib.tm_ce_grad_h_bf16(out.data_ptr(), a.data_ptr(), wt.data_ptr(), rows, vocab, dim,
                                       ws.data_ptr(), nbytes, stream), "tm_ce_grad_h_bf16")
    return out


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (x in fp64): 2^(e - 7) for |x| in [2^e, 2^(e+1))."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("rows,cols", [(64, 64), (128, 192), (151936, 1024)])
def test_transpose_is_exact(rows, cols):
    g = torch.Generator(device=DEV).manual_seed(rows + cols)
    w = torch.randn(rows, cols, device=DEV, generator=g).to(torch.bfloat16)
    wt = _transpose(w)
    torch.cuda.synchronize()
    assert torch.equal(wt.view(torch.int16), w.t().contiguous().view(torch.int16))


@pytest.mark.parametrize("rows,vocab,dim,softmax", [
    (256, 640, 256, False),        # one tile, 256 splits over 10 K slices: most splits empty
    (256, 4096, 512, False),
    (512, 2048, 768, True),
    (1024, 151936, 1024, True),    # the Qwen3-0.6B head at the reference's 1024-row chunk
    (2048, 32768, 1024, False),
    (4096, 8192, 2560, True),      # a 4096-row chunk of the Qwen3-4B width
])
def test_grad_h_gemm_vs_fp64_and_library(rows, vocab, dim, softmax):
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + vocab + dim)
    if softmax:  # grad_logits as the row kernel writes them: softmax - onehot on most rows
        x = torch.randn(rows, vocab, device=DEV, generator=g) * 3.0
        p = torch.softmax(x, dim=1)
        lab = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
        p[torch.arange(rows, device=DEV), lab] -= 1.0
        p[::9] = 0.0  # ignored rows
        a = p.to(torch.bfloat16)
        del x, p
    else:
        a = torch.randn(rows, vocab, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(vocab, dim, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    out = _grad_h(a, w)
    exact = torch.matmul(a.double(), w.double())
    absum = torch.matmul(a.double().abs(), w.double().abs())
    lib_out = torch.matmul(a, w)
    torch.cuda.synchronize()
    err = (out.double() - exact).abs()
    bound = _bf16_ulp(exact) + absum * 2.0 ** -20
    worst = float((err / bound).max())
    print(f"{rows}x{vocab}x{dim}: worst |err| / bound {worst:.3f}")
    assert worst <= 1.0
    d = (out.double() - lib_out.double()).abs()
    assert bool((d <= _bf16_ulp(torch.maximum(out.double().abs(), lib_out.double().abs())) + absum * 2.0 ** -19).all())
    same = float((out.view(torch.int16) == lib_out.view(torch.int16)).double().mean())
    print(f"  equal to torch.matmul on {same:.5f} of the elements")
    assert same >= 0.99


def test_grad_h_gemm_is_deterministic():
    g = torch.Generator(device=DEV).manual_seed(5)
    a = torch.randn(1024, 16384, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.randn(16384, 1024, device=DEV, generator=g).to(torch.bfloat16)
    first = _grad_h(a, w)
    again = _grad_h(a, w, ws_fill=0x7F)  # workspace full of other data (3.4e38)
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("chunk", [1024, 768, None])
def test_op_grad_h_uses_the_gemm_on_eligible_chunks(chunk):
    """grad_h of the op on chunks of 1024, 768 and 3072 rows (3072 rows, D 256, V 4096): every
    chunk's grad_h equals tm_ce_grad_h_bf16 on that chunk's grad_logits, times the bf16 scale,
    bit for bit, and loss and both gradients stay within the reference composition's bars."""
    from torchure_amd import _native
    from torchure_amd.loss import fused_linear_cross_entropy
    from torchure_amd.loss.fused_linear_ce import splitk_grad_h_fits

    g = torch.Generator(device=DEV).manual_seed(31)
    n, d, v = 3072, 256, 4096
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::19] = -100
    h1 = hidden.clone().requires_grad_(True)
    w1 = weight.clone().requires_grad_(True)
    loss = fused_linear_cross_entropy(h1, w1, labels, -100, chunk)
    loss.backward()

    lib, stream = _native.lib(), _native.stream_handle(DEV)
    w = weight.to(torch.bfloat16)
    step = chunk or n
    want = torch.empty_like(hidden)
    row_loss = torch.empty(n, dtype=torch.float32, device=DEV)
    for s in range(0, n, step):
        e = min(s + step, n)
        assert splitk_grad_h_fits(e - s, d, v)
        logits = torch.matmul(hidden[s:e], w.t())
        _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v, -100,
                                          row_loss[s:].data_ptr(), stream), "tm_ce_rows_bf16")
        want[s:e] = _grad_h(logits, w)
    n_valid = (labels != -100).sum().clamp_min(1)
    want.mul_((torch.tensor(1.0, device=DEV) / n_valid).to(torch.bfloat16))
    ref_loss, ref_gh, ref_gw = fused_linear_ce_reference(hidden, weight, labels, -100, chunk_size=step)
    torch.cuda.synchronize()
    assert torch.equal(h1.grad.view(torch.int16), want.view(torch.int16))
    assert abs(loss.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
    assert (h1.grad.float() - ref_gh.float()).abs().max().item() <= 1e-2 * ref_gh.float().abs().max().item()
    assert (w1.grad - ref_gw).abs().max().item() <= 1e-2 * ref_gw.abs().max().item()


def test_op_mixes_the_gemm_and_the_library_on_ragged_chunks():
    """2600 rows in 1024-row chunks (D 256, V 4096): the two full chunks take the split-K
    GEMM and the 552-row tail torch.matmul, each bit for bit, within one call."""
    from torchure_amd import _native
    from torchure_amd.loss import fused_linear_cross_entropy
    from torchure_amd.loss.fused_linear_ce import splitk_grad_h_fits

    g = torch.Generator(device=DEV).manual_seed(41)
    n, d, v, chunk = 2600, 256, 4096, 1024
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::23] = -100
    h1 = hidden.clone().requires_grad_(True)
    fused_linear_cross_entropy(h1, weight, labels, -100, chunk).backward()

    lib, stream = _native.lib(), _native.stream_handle(DEV)
    w = weight.to(torch.bfloat16)
    want = torch.empty_like(hidden)
    row_loss = torch.empty(n, dtype=torch.float32, device=DEV)
    kinds = []
    for s in range(0, n, chunk):
        e = min(s + chunk, n)
        logits = torch.matmul(hidden[s:e], w.t())
        _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v, -100,
                                          row_loss[s:].data_ptr(), stream), "tm_ce_rows_bf16")
        fits = splitk_grad_h_fits(e - s, d, v)
        kinds.append(fits)
        want[s:e] = _grad_h(logits, w) if fits else torch.matmul(logits, w)
    assert kinds == [True, True, False]
    n_valid = (labels != -100).sum().clamp_min(1)
    want.mul_((torch.tensor(1.0, device=DEV) / n_valid).to(torch.bfloat16))
    torch.cuda.synchronize()
    assert torch.equal(h1.grad.view(torch.int16), want.view(torch.int16))
