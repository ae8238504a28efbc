"""GPU parity of the fused CE's three bf16 MFMA GEMMs (torchure/loss/fused_linear_ce.py:38,52,57):
tm_ce_logits_bf16 (logits = h W^T), tm_ce_grad_h_bf16 (split-K grad_h = grad_logits W) and
tm_ce_grad_w_bf16 (grad_W = grad_logits^T h).

Checks:
- each GEMM against an fp64 product of the same bf16 operands: every element within one bf16
  ulp of the exact value plus 2^-20 of sum_k |a_ik b_kj| (the fp32 accumulation), at shapes
  from one tile (or one K slice per split) with ragged edges up to the Qwen3 heads' chunks;
- against torch.matmul (hipBLASLt) on the same operands: within one bf16 ulp plus the two
  fp32 accumulation budgets everywhere, and equal on at least 99% of the elements (the two
  differ only in fp32 summation order);
- deterministic: the same bits on a repeat call (for grad_h over a workspace holding other
  data); no write outside the output;
- the persistent logits and grad_W kernels against the one-tile-per-workgroup kernels on the
  same products: the same bits;
- inside the op: the fused CE's grad_h equals the chosen GEMM's result for the chunk's
  grad_logits, and the whole op stays within the reference composition's bars.
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


def _grad_h(a, w, ws_fill=None):
    native, lib, stream = _lib()
    rows, vocab = a.shape
    dim = w.shape[1]
    nbytes = lib.tm_ce_grad_h_workspace_bytes(rows, vocab, dim)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    if ws_fill is not None:
        ws.fill_(ws_fill)
    out = torch.empty((rows, dim), dtype=torch.bfloat16, device=DEV)
    native.check(lib.tm_ce_grad_h_bf16(out.data_ptr(), a.data_ptr(), w.data_ptr(), rows, vocab, dim,
                                       ws.data_ptr(), nbytes, stream), "tm_ce_grad_h_bf16")
    return out


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (x in fp64): 2^(e - 7) for |x| in [2^e, 2^(e+1))."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


@pytest.mark.parametrize("rows,vocab,dim,softmax", [
    (256, 640, 256, False),        # one tile, 10 splits of one K slice each
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
        logits, _ = _logits(hidden[s:e], w)  # the op's logits GEMM
        logits = logits.contiguous()
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
        logits, _ = _logits(hidden[s:e], w)  # the op's logits GEMM
        logits = logits.contiguous()
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


@pytest.mark.parametrize("d,split", [(768, True), (1024, False)])
def test_op_grad_h_choice_above_64_tiles(d, split):
    """One 8192-row chunk (V 4096): at a hidden size that is not a power of two (768, 96 output
    tiles) grad_h takes the split-K GEMM, at a power of two (1024, 128 tiles) torch.matmul; the
    op's grad_h equals the chosen product times the bf16 scale, bit for bit."""
    from torchure_amd import _native
    from torchure_amd.loss import fused_linear_cross_entropy
    from torchure_amd.loss.fused_linear_ce import splitk_grad_h_fits

    g = torch.Generator(device=DEV).manual_seed(d)
    n, v = 8192, 4096
    assert splitk_grad_h_fits(n, d, v) == split
    hidden = torch.randn(n, d, device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=DEV, generator=g) * 0.05
    labels = torch.randint(0, v, (n,), device=DEV, generator=g)
    labels[::17] = -100
    h1 = hidden.clone().requires_grad_(True)
    fused_linear_cross_entropy(h1, weight, labels, -100, None).backward()

    lib, stream = _native.lib(), _native.stream_handle(DEV)
    w = weight.to(torch.bfloat16)
    logits, _ = _logits(hidden, w)  # the op's logits GEMM
    logits = logits.contiguous()
    row_loss = torch.empty(n, dtype=torch.float32, device=DEV)
    _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), v, labels.data_ptr(), n, v, -100, row_loss.data_ptr(),
                                      stream), "tm_ce_rows_bf16")
    want = _grad_h(logits, w) if split else torch.matmul(logits, w)
    n_valid = (labels != -100).sum().clamp_min(1)
    want.mul_((torch.tensor(1.0, device=DEV) / n_valid).to(torch.bfloat16))
    torch.cuda.synchronize()
    assert torch.equal(h1.grad.view(torch.int16), want.view(torch.int16))


def _logits(h, w, pad=64, sentinel=0x7BCD):
    """tm_ce_logits_bf16 into a view with `pad` guard elements on both sides (sentinel bits),
    returning (logits, guard intact)."""
    native, lib, stream = _lib()
    rows, vocab = h.shape[0], w.shape[0]
    buf = torch.full((rows * vocab + 2 * pad,), sentinel, dtype=torch.int16, device=DEV)
    out = buf[pad: pad + rows * vocab].view(torch.bfloat16).view(rows, vocab)
    native.check(lib.tm_ce_logits_bf16(out.data_ptr(), h.data_ptr(), w.data_ptr(), rows, vocab, h.shape[1], stream),
                 "tm_ce_logits_bf16")
    torch.cuda.synchronize()
    guard = bool((buf[:pad] == sentinel).all()) and bool((buf[pad + rows * vocab:] == sentinel).all())
    return out, guard


@pytest.mark.parametrize("rows,vocab,dim", [
    (1, 1, 64),              # one element
    (7, 100, 64),            # vocab not a multiple of 8: element-wise stores
    (255, 4095, 128),        # rows and vocab one short of tile multiples
    (257, 4097, 128),        # one past: mostly empty edge tiles
    (1000, 1001, 192),
    (300, 1000, 256),        # persistent kernel from here: 4 K slices (its minimum), ragged edges
    (64, 200, 256),          # one tile: one workgroup works, the rest exit at once
    (2000, 20008, 384),      # 6 K slices; edge tiles in both directions
    (8200, 4104, 512),       # several tiles per workgroup, a 9-row last tile row
    (1024, 151936, 1024),    # the Qwen3-0.6B head at the reference's 1024-row chunk
    (4096, 151936, 1024),
    (1500, 32768, 2560),     # Qwen3-4B width, ragged rows
])
def test_logits_gemm_vs_fp64_and_library(rows, vocab, dim):
    """logits = h @ W^T (fused_linear_ce.py:38) on this build's GEMM: every element within one
    bf16 ulp of the exact product of the same bf16 operands plus 2^-20 of sum_k |h_ik w_jk| (the
    fp32 accumulation), within one ulp plus both budgets of torch.matmul's, equal to it on at
    least 99% of the elements, no write outside the output, and the same bits on a repeat."""
    g = torch.Generator(device=DEV).manual_seed(rows * 3 + vocab + dim)
    h = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(vocab, dim, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    out, guard = _logits(h, w)
    assert guard
    exact = torch.matmul(h.double(), w.double().t())
    absum = torch.matmul(h.double().abs(), w.double().abs().t())
    lib_out = torch.matmul(h, w.t())
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
    again, _ = _logits(h, w)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_logits_gemm_full_chunk_vs_library():
    """The whole 8192-token Qwen3-0.6B head in one chunk (the op's MI355X sizing): against
    torch.matmul row block by row block, within one bf16 ulp plus both fp32 budgets, equal on
    at least 99% of the elements."""
    rows, vocab, dim = 8192, 151936, 1024
    g = torch.Generator(device=DEV).manual_seed(8192)
    h = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(vocab, dim, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    out, guard = _logits(h, w)
    assert guard
    same = 0.0
    for s in range(0, rows, 1024):
        lib_out = torch.matmul(h[s:s + 1024], w.t())
        o = out[s:s + 1024]
        absum = torch.matmul(h[s:s + 1024].float().abs(), w.float().abs().t()).double()
        d = (o.double() - lib_out.double()).abs()
        assert bool((d <= _bf16_ulp(torch.maximum(o.double().abs(), lib_out.double().abs())) + absum * 2.0 ** -19).all())
        same += float((o.view(torch.int16) == lib_out.view(torch.int16)).double().mean()) / (rows // 1024)
    print(f"equal to torch.matmul on {same:.5f} of the elements")
    assert same >= 0.99


@pytest.mark.parametrize("rows,vocab,dim", [
    (300, 1000, 256),
    (2000, 20008, 384),
    (1500, 32768, 2560),
    (1024, 151936, 1024),
    (8192, 151936, 1024),
])
def test_logits_ring_kernel_equals_one_tile_kernel(rows, vocab, dim):
    """The persistent logits kernel (vocab a multiple of 8) and the one-tile-per-workgroup kernel
    give the same bits: with one more weight row the vocabulary is no longer a multiple of 8, the
    call takes the one-tile kernel, and every element of the first `vocab` columns keeps its
    tile, its lanes and its MFMA sequence."""
    g = torch.Generator(device=DEV).manual_seed(rows + vocab + 7 * dim)
    h = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(vocab + 1, dim, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    ring, guard = _logits(h, w1[:vocab])
    assert guard
    tile, guard = _logits(h, w1)
    assert guard
    assert torch.equal(ring.view(torch.int16), tile[:, :vocab].view(torch.int16))


def test_logits_gemm_argument_checks():
    """Shapes the GEMM does not take and misaligned pointers are refused before any launch."""
    native, lib, stream = _lib()
    t = torch.empty(1 << 16, dtype=torch.bfloat16, device=DEV)
    p = t.data_ptr()
    for rows, vocab, dim in ((0, 64, 64), (64, 0, 64), (64, 64, 100), (64, 64, 0)):
        assert lib.tm_ce_logits_bf16(p, p, p, rows, vocab, dim, stream) < 0
    assert lib.tm_ce_logits_bf16(p + 2, p, p, 8, 8, 64, stream) < 0
    assert b"aligned" in lib.tm_last_error()


def _grad_w(gl, h, pad=64, sentinel=0x7BCD):
    """tm_ce_grad_w_bf16 into a view with guard elements on both sides."""
    native, lib, stream = _lib()
    rows, vocab = gl.shape
    dim = h.shape[1]
    buf = torch.full((vocab * dim + 2 * pad,), sentinel, dtype=torch.int16, device=DEV)
    out = buf[pad: pad + vocab * dim].view(torch.bfloat16).view(vocab, dim)
    native.check(lib.tm_ce_grad_w_bf16(out.data_ptr(), gl.data_ptr(), h.data_ptr(), rows, vocab, dim, stream),
                 "tm_ce_grad_w_bf16")
    torch.cuda.synchronize()
    guard = bool((buf[:pad] == sentinel).all()) and bool((buf[pad + vocab * dim:] == sentinel).all())
    return out, guard


@pytest.mark.parametrize("rows,vocab,dim,softmax", [
    (64, 8, 8, False),            # one K stage, one tile mostly past vocab and dim
    (128, 4104, 264, False),      # vocab and dim one group of 8 past tile multiples
    (192, 1000, 136, True),
    (256, 1000, 256, True),       # persistent kernel from here: 4 K stages (its minimum), ragged vocab
    (384, 4104, 520, False),      # 6 K stages; edge tiles in both directions
    (512, 200, 264, True),        # 2 tiles: most workgroups exit at once
    (1024, 151936, 1024, True),   # the Qwen3-0.6B head at the reference's 1024-row chunk
    (4096, 32768, 2560, True),    # a 4096-row chunk at the Qwen3-4B width
])
def test_grad_w_gemm_vs_fp64_and_library(rows, vocab, dim, softmax):
    """A chunk's gw = grad_logits^T @ h (fused_linear_ce.py:57) on this build's transposed-read
    GEMM: every element within one bf16 ulp of the exact product of the same bf16 operands plus
    2^-20 of sum_k |g_kv h_kd|, within one ulp plus both budgets of torch.matmul's, equal to it
    on at least 99% of the elements, no write outside the output, the same bits on a repeat."""
    g = torch.Generator(device=DEV).manual_seed(rows + vocab * 5 + dim)
    if softmax:  # grad_logits as the row kernel writes them
        x = torch.randn(rows, vocab, device=DEV, generator=g) * 3.0
        p = torch.softmax(x, dim=1)
        lab = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
        p[torch.arange(rows, device=DEV), lab] -= 1.0
        p[::7] = 0.0
        gl = p.to(torch.bfloat16)
        del x, p
    else:
        gl = torch.randn(rows, vocab, device=DEV, generator=g).to(torch.bfloat16)
    h = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    out, guard = _grad_w(gl, h)
    assert guard
    exact = torch.matmul(gl.double().t(), h.double())
    absum = torch.matmul(gl.double().abs().t(), h.double().abs())
    lib_out = torch.matmul(gl.t(), h)
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
    again, _ = _grad_w(gl, h)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_grad_w_gemm_full_chunk_vs_library():
    """The 8192-row chunk of the Qwen3-0.6B head (the op's MI355X sizing): against torch.matmul,
    within one bf16 ulp plus both fp32 budgets, equal on at least 99% of the elements."""
    rows, vocab, dim = 8192, 151936, 1024
    g = torch.Generator(device=DEV).manual_seed(81920)
    gl = (torch.randn(rows, vocab, device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
    h = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    out, guard = _grad_w(gl, h)
    assert guard
    lib_out = torch.matmul(gl.t(), h)
    same = 0.0
    for s in range(0, vocab, 16384):
        e = min(s + 16384, vocab)
        absum = torch.matmul(gl[:, s:e].float().abs().t(), h.float().abs()).double()
        o, l_ = out[s:e].double(), lib_out[s:e].double()
        assert bool(((o - l_).abs() <= _bf16_ulp(torch.maximum(o.abs(), l_.abs())) + absum * 2.0 ** -19).all())
        same += float((out[s:e].view(torch.int16) == lib_out[s:e].view(torch.int16)).double().sum())
    same /= vocab * dim
    print(f"equal to torch.matmul on {same:.5f} of the elements")
    assert same >= 0.99


@pytest.mark.parametrize("rows,vocab,dim", [
    (256, 1000, 256),
    (384, 4104, 520),
    (1024, 151936, 1024),
    (4096, 32768, 2560),
    (8192, 151936, 1024),
])
def test_grad_w_ring_kernel_equals_one_tile_kernel(rows, vocab, dim):
    """The persistent grad_W kernel (rows a multiple of 128) and the one-tile-per-workgroup
    kernel give the same values: 64 zero rows appended to grad_logits (and any 64 rows to h) make
    the call take the one-tile kernel with one more K slice, whose products are all zero, so every
    sum is the same; only the sign of an exact zero could differ, which a value comparison
    ignores."""
    g = torch.Generator(device=DEV).manual_seed(rows * 11 + vocab + dim)
    x = torch.randn(rows, vocab, device=DEV, generator=g) * 3.0
    p = torch.softmax(x, dim=1)
    del x
    lab = torch.randint(0, vocab, (rows,), device=DEV, generator=g)
    p[torch.arange(rows, device=DEV), lab] -= 1.0
    gl = torch.zeros(rows + 64, vocab, dtype=torch.bfloat16, device=DEV)
    gl[:rows] = p.to(torch.bfloat16)
    del p
    h = torch.randn(rows + 64, dim, device=DEV, generator=g).to(torch.bfloat16)
    ring, guard = _grad_w(gl[:rows], h[:rows])
    assert guard
    tile, guard = _grad_w(gl, h)
    assert guard
    assert torch.equal(ring, tile)


def test_grad_w_gemm_argument_checks():
    """Row counts off a multiple of 64, vocab or dim off a multiple of 8 and misaligned pointers
    are refused before any launch."""
    native, lib, stream = _lib()
    t = torch.empty(1 << 16, dtype=torch.bfloat16, device=DEV)
    p = t.data_ptr()
    for rows, vocab, dim in ((0, 64, 64), (100, 64, 64), (64, 60, 64), (64, 64, 60), (64, 0, 64)):
        assert lib.tm_ce_grad_w_bf16(p, p, p, rows, vocab, dim, stream) < 0
    assert lib.tm_ce_grad_w_bf16(p + 2, p, p, 64, 8, 8, stream) < 0
    assert b"aligned" in lib.tm_last_error()
