"""Chunked fused linear + cross-entropy on gfx950.

Same function, arguments and semantics as torchure/loss/fused_linear_ce.py:130-136:
``fused_linear_cross_entropy(hidden, weight, labels, ignore_index=-100, chunk_size=...)``
returns the mean loss over non-ignored tokens (F.cross_entropy(reduction="mean")
semantics, :22-24), computes grad_hidden and grad_weight during the forward pass
(:42-58) and scales them in place by grad_out / n_valid in backward (:94-127).

Per chunk of rows:
  logits = h @ W^T                  bf16 GEMM: tm_ce_logits_bf16, this build's MFMA GEMM, for dim a
                                    multiple of 64 (torch.matmul on other shapes)
  tm_ce_rows_bf16                   one fused kernel: logsumexp, per-row loss and
                                    grad_logits = bf16(softmax - onehot), in place
  grad_h = grad_logits @ W          bf16 GEMM: tm_ce_grad_h_bf16, a split-K MFMA GEMM with a
                                    fixed-order reduction, on chunks with at most
                                    SPLITK_GRAD_H_MAX_TILES output tiles of 256 x 256, or any
                                    number when D is not a power of two (rows and D multiples of
                                    256, V of 64); hipBLASLt on other shapes
  grad_W += grad_logits^T @ h       bf16 GEMM: tm_ce_grad_w_bf16, this build's MFMA GEMM, for rows a
                                    multiple of 64 (torch.matmul on other shapes), then
                                    tm_ce_grad_w_fold into fp32
then tm_ce_loss sums the per-row losses in a fixed order (deterministic).

The last chunk's bf16 grad_W is not added in forward: it waits for backward, where
tm_ce_grad_w adds it and applies grad_out / n_valid in the same pass. With a single
chunk (the usual case at 4 GiB of logits) the fp32 grad_W is then written once,
straight from the bf16 GEMM output (6 B per element), instead of a zero fill, an
accumulate and a scaling pass (22 B per element). With several chunks, the chunks'
bf16 grad_W wait and are added up to 8 at a time (tm_ce_grad_w_fold: one read and one
write of the fp32 grad_W per fold; a fold also starts once 4 GiB of chunks wait), and the
chunks still waiting are added together with the last in backward. The fp32 additions and
the scaling are the reference's, in the reference's order, so the bits are unchanged.

Only the gradients autograd needs are computed. With grad mode off, or no input that
requires a gradient (evaluation), the call returns the loss from the logits GEMM and
tm_ce_rows_loss_bf16, which runs the same per-row arithmetic without the gradient
write, so the loss bits are those of the training path. When only one input requires a
gradient, the other's GEMM is skipped. The reference computes both gradients whenever
the weight requires one (fused_linear_ce.py:63-93) and lets autograd drop them.

Hidden states are bf16 or fp32. fp32 inside bf16 CUDA autocast is the trainer's call
(objectives/autoregressive.py:38-44): it passes the final norm's fp32 output, for which the
reference's buffers take fp32 (:65,68) and autocast runs the products on bf16 casts. Here
hidden is cast to bf16 once (RNE, as autocast does), grad_hidden stays a bf16 GEMM output
until backward, and tm_ce_widen_scale writes the fp32 gradient float(gh) * grad_out / n_valid
(the reference's fp32 copy and mul_, :80,120). fp32 hidden states outside autocast take the
reference's fp32 path: fp32 GEMMs on weight.to(fp32), tm_ce_rows_f32 on fp32 logits, and the
reference's fp32 `+=` and `mul_` for grad_W.

Chunking: 1024 rows by default, the reference's default (:131). ``chunk_size=None`` or
``"auto"`` opts into MI355X sizing: chunks whose bf16 logits take up to 4 GiB, so that
with 288 GB of HBM the whole Qwen3 vocabulary for 8K-16K tokens fits in one chunk, the
fp32 grad_W is written once, by the backward hand-over, instead of being read and written
for every fold of 1024-row chunks, and the GEMMs get large M.
"""

from __future__ import annotations

import contextlib
import ctypes
import threading

import torch

from torchure_amd import _native
from torchure_amd.core import tables
from torchure_amd.optimizer.working import current_copy

DEFAULT_LOGITS_BYTES = 4 << 30


class CallOrder:
    """Puts the GPU work of this op's calls on one device in host call order.

    hipBLASLt's gfx950 solutions for this op's products are stream-K kernels (``SK3`` in
    their names): a persistent grid of one workgroup per CU in which workgroups spin on
    flags until other workgroups of the same launch have written their partial tiles, so
    every workgroup of the launch must be resident at once. Two such launches running at
    the same time on two streams can each hold CUs with spinning workgroups while the
    workgroups they wait for cannot be placed, and neither finishes. So each call's stream
    first waits for an event recorded at the end of the previous call's GPU work on that
    device (skipped when both run on one stream), and the host side of a call runs under a
    lock, so that calls from two host threads cannot interleave either. The event is
    always recorded before the next call waits on it, so a wait never sits in front of the
    work that signals it. GEMMs that a caller runs on other streams are not ordered by
    this; they must not overlap a call.

    ``current_stream`` and ``make_event`` are injectable so the ordering can be checked on
    the CPU with stand-in streams and events."""

    def __init__(self, current_stream=None, make_event=None):
        self._current_stream = current_stream or torch.cuda.current_stream
        self._make_event = make_event or torch.cuda.Event
        self._lock = threading.RLock()
        self._last: dict = {}  # device index -> (stream, event) of the last call there

    @contextlib.contextmanager
    def call(self, device: torch.device):
        if device.type != "cuda":  # the call raises on its argument checks; nothing to order
            yield None
            return
        key = device.index if device.index is not None else -1
        with self._lock:
            stream = self._current_stream(device)
            prev = self._last.get(key)
            if prev is not None and prev[0] != stream:
                stream.wait_event(prev[1])
            try:
                yield stream
            finally:
                done = self._make_event()
                done.record(stream)
                self._last[key] = (stream, done)


CALL_ORDER = CallOrder()


def auto_chunk_rows(n_rows: int, vocab: int, logits_bytes: int = DEFAULT_LOGITS_BYTES) -> int:
    rows = max(256, logits_bytes // (2 * vocab) // 256 * 256)
    return max(1, min(n_rows, rows))


def _fp32_hidden_under_autocast(hidden) -> bool:
    """fp32 hidden states inside bf16 CUDA autocast: the reference trainer's call (its final
    RMSNorm leaves the fp32 residual stream in fp32), where autocast runs the op's products as
    bf16 GEMMs and the hidden-state gradient stays fp32."""
    return (hidden.dtype == torch.float32 and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16)


def _checked(hidden, weight, labels, chunk_size):
    """Argument checks shared by all paths; returns (n, v, chunk rows, mode): "bf16" (bf16
    hidden), "autocast" (fp32 hidden inside bf16 autocast: bf16 products) or "fp32" (fp32 hidden
    outside autocast: fp32 products, as the reference's with w = weight.to(fp32))."""
    who = "fused_linear_cross_entropy"
    for t, what in ((hidden, "hidden"), (labels, "labels")):  # made contiguous by the caller
        tables.require_device_tensor(t, who, what)
    if weight.device.type != "cuda":  # any strides: the op works on its contiguous bf16 cast
        raise RuntimeError(f"{who}: weight must be on a ROCm GPU device, got {weight.device} "
                           "(torchure_amd has no CPU path)")
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") != torch.bfloat16:
        # autocast would run the products in its dtype (the reference's GEMMs too), and the
        # row kernel reads bf16 logits
        raise NotImplementedError(
            f"{who}: CUDA autocast with {torch.get_autocast_dtype('cuda')} is not supported; the "
            "products run as bf16 GEMMs (bf16 autocast, or none)")
    if _fp32_hidden_under_autocast(hidden):
        mode = "autocast"
    elif hidden.dtype == torch.float32 and not torch.is_autocast_enabled("cuda"):
        mode = "fp32"
    elif hidden.dtype == torch.bfloat16:
        mode = "bf16"
    else:
        raise NotImplementedError(
            f"{who}: hidden must be bfloat16, or float32 (inside bf16 CUDA autocast or outside autocast), "
            f"got {hidden.dtype} with autocast " + ("on" if torch.is_autocast_enabled("cuda") else "off"))
    if labels.dtype != torch.int64:
        raise RuntimeError(f"{who}: labels must be int64")
    n, d = hidden.shape
    v = weight.shape[0]
    if weight.shape[1] != d or labels.shape[0] != n:
        raise RuntimeError(f"{who}: shapes hidden {tuple(hidden.shape)}, weight {tuple(weight.shape)}, "
                           f"labels {tuple(labels.shape)} do not match")
    if weight.device != hidden.device or labels.device != hidden.device:
        raise RuntimeError(f"{who}: hidden, weight and labels must be on one device")
    auto = chunk_size is None or (isinstance(chunk_size, str) and chunk_size == "auto")
    if isinstance(chunk_size, str) and not auto:
        raise ValueError(f"{who}: chunk_size must be a positive int, None or 'auto', got {chunk_size!r}")
    chunk = auto_chunk_rows(n, v) if auto else int(chunk_size)
    if chunk < 1:
        raise ValueError(f"{who}: chunk_size must be positive, got {chunk_size}")
    return n, v, chunk, mode


def _bf16(logits: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """The row kernels read bf16 bits (fp32 on the fp32 path): refuse anything else loudly."""
    if logits.dtype != dtype or not logits.is_contiguous():
        raise RuntimeError(f"fused_linear_cross_entropy: the logits GEMM returned {logits.dtype} "
                           f"(contiguous: {logits.is_contiguous()}), the row kernels need contiguous {dtype}")
    return logits


def _mean_loss(row_loss, labels, n, ignore_index, lib, stream):
    """(mean loss as a 0-d tensor, n_valid as a 1-element view) from the per-row losses."""
    out3 = torch.empty(3, dtype=torch.float32, device=row_loss.device)
    _native.check(lib.tm_ce_loss(row_loss.data_ptr(), labels.data_ptr(), n, int(ignore_index),
                                 out3.data_ptr(), stream), "tm_ce_loss")
    return out3[2].clone(), out3[1:2]


def logits_gemm_fits(h: torch.Tensor, w: torch.Tensor) -> bool:
    """Chunks whose logits run on this build's GEMM (tm_ce_logits_bf16): bf16 operands, both
    contiguous and 16-byte aligned, dim a multiple of 64. Other shapes take torch.matmul."""
    return (h.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and h.dim() == 2 and w.dim() == 2
            and h.shape[1] == w.shape[1] and h.shape[1] % 64 == 0 and h.shape[0] > 0 and w.shape[0] > 0
            and h.is_contiguous() and w.is_contiguous() and h.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)


def _logits(h: torch.Tensor, w: torch.Tensor, lib, stream) -> torch.Tensor:
    """logits = h @ w.T (fused_linear_ce.py:38): a bf16 GEMM, fp32 accumulation, bf16 result."""
    if not logits_gemm_fits(h, w):
        return _bf16(torch.matmul(h, w.t()))
    rows, dim = h.shape
    out = torch.empty((rows, w.shape[0]), dtype=torch.bfloat16, device=h.device)
    _native.check(lib.tm_ce_logits_bf16(out.data_ptr(), h.data_ptr(), w.data_ptr(), rows, w.shape[0], dim, stream),
                  "tm_ce_logits_bf16")
    return out


def grad_w_gemm_fits(g: torch.Tensor, h: torch.Tensor) -> bool:
    """Chunks whose grad_W runs on this build's GEMM (tm_ce_grad_w_bf16): bf16 operands, both
    contiguous and 16-byte aligned, rows a multiple of 64, vocab and dim multiples of 8. Other
    shapes take torch.matmul."""
    return (g.dtype == torch.bfloat16 and h.dtype == torch.bfloat16 and g.dim() == 2 and h.dim() == 2
            and g.shape[0] == h.shape[0] and g.shape[0] > 0 and g.shape[0] % 64 == 0 and g.shape[1] % 8 == 0
            and h.shape[1] % 8 == 0 and g.shape[1] > 0 and h.shape[1] > 0 and g.is_contiguous() and h.is_contiguous()
            and g.data_ptr() % 16 == 0 and h.data_ptr() % 16 == 0)


def _grad_w(g: torch.Tensor, h: torch.Tensor, lib, stream) -> torch.Tensor:
    """A chunk's gw = grad_logits.t() @ h (fused_linear_ce.py:57): bf16 GEMM, bf16 result (V x D)."""
    if not grad_w_gemm_fits(g, h):
        return torch.matmul(g.t(), h)
    rows, vocab = g.shape
    out = torch.empty((vocab, h.shape[1]), dtype=torch.bfloat16, device=g.device)
    _native.check(lib.tm_ce_grad_w_bf16(out.data_ptr(), g.data_ptr(), h.data_ptr(), rows, vocab, h.shape[1], stream),
                  "tm_ce_grad_w_bf16")
    return out


SPLITK_GRAD_H_MAX_TILES = 64


def splitk_grad_h_fits(rows: int, dim: int, vocab: int) -> bool:
    """Chunks whose grad_h runs on the split-K MFMA GEMM (tm_ce_grad_h_bf16): the shapes it
    tiles (rows and dim multiples of 256, vocab of 64), except where the library GEMM measured
    faster on MI355X: more than SPLITK_GRAD_H_MAX_TILES output tiles of 256 x 256 with dim a
    power of two. With few tiles and K = vocab a library GEMM leaves most of the 256 CUs idle and
    the split-K kernel spreads K over them; with many, the library's kernels fill the chip
    themselves, and beat this kernel by 1.5-7% when dim is a power of two, but run 12-50% behind
    it at the other Qwen3 head widths (ms per call at V = 151,936, split-K / hipBLASLt):

        dim   rows 1024      2048           4096           8192
        1024  0.30 / 0.78    0.65 / 1.08    1.07 / 1.51    2.11 / 2.08
        2048  0.55 / 0.90    1.04 / 1.65    2.06 / 2.01    4.11 / 3.95
        2560  0.69 / 1.03    1.35 / 1.90    2.82 / 3.52    5.42 / 7.40
        4096  1.07 / 1.88    2.11 / 2.03    4.16 / 3.88    8.35 / 7.76
        5120  1.43 / 1.89    3.11 / 3.48    5.70 / 7.07    11.34 / 13.41
    """
    if not (rows > 0 and dim > 0 and rows % 256 == 0 and dim % 256 == 0 and dim <= 65536
            and vocab > 0 and vocab % 64 == 0):
        return False
    return (rows // 256) * (dim // 256) <= SPLITK_GRAD_H_MAX_TILES or (dim & (dim - 1)) != 0


FOLD_CHUNKS = 8  # chunks per grad_W fold (tm_ce_grad_w_fold takes at most 8)
FOLD_BYTES = 4 << 30  # bf16 chunk grad_W held before a fold, at most


def _fold(lib, grad_weight, chunks, accumulated, g, n_valid, stream) -> None:
    """grad_weight = ((grad_weight or +0) + float(c0) + float(c1) + ...) [* g / n_valid], the
    reference's `grad_weight += gw` per chunk in order (fused_linear_ce.py:80-81) and, with g,
    its backward `mul_` (:126), in one pass over the fp32 buffer."""
    ptrs = (ctypes.c_void_p * len(chunks))(*[c.data_ptr() for c in chunks])
    _native.check(lib.tm_ce_grad_w_fold(grad_weight.data_ptr(), ptrs, len(chunks), chunks[0].numel(),
                                        int(accumulated), g.data_ptr() if g is not None else None,
                                        n_valid.data_ptr() if n_valid is not None else None, stream),
                  "tm_ce_grad_w_fold")


class GradHidden:
    """grad_h = grad_logits @ W (fused_linear_ce.py:52, stored at :79) for the chunks of one
    call: the split-K MFMA GEMM on the chunks ``splitk_grad_h_fits`` accepts, reading W as it is
    stored, with one fp32 partials workspace shared by the chunks (stream-ordered), and
    torch.matmul (hipBLASLt) on the others. ``w`` is the contiguous bf16 weight (V x D)."""

    def __init__(self, w: torch.Tensor, chunk_rows, lib, stream):
        self.w, self.lib, self.stream = w, lib, stream
        self.vocab, self.dim = w.shape
        fits = [r for r in set(chunk_rows) if splitk_grad_h_fits(r, self.dim, self.vocab)]
        self.ws = None
        if fits:
            nbytes = max(lib.tm_ce_grad_h_workspace_bytes(r, self.vocab, self.dim) for r in fits)
            self.ws = torch.empty(nbytes, dtype=torch.uint8, device=w.device)

    def __call__(self, grad_logits: torch.Tensor, out: torch.Tensor) -> None:
        rows = grad_logits.shape[0]
        if self.ws is None or not splitk_grad_h_fits(rows, self.dim, self.vocab):
            torch.matmul(grad_logits, self.w, out=out)
            return
        if not (grad_logits.is_contiguous() and out.is_contiguous() and out.dtype == torch.bfloat16):
            raise RuntimeError("fused_linear_cross_entropy: grad_h GEMM operands must be contiguous bf16")
        _native.check(self.lib.tm_ce_grad_h_bf16(out.data_ptr(), grad_logits.data_ptr(), self.w.data_ptr(), rows,
                                                 self.vocab, self.dim, self.ws.data_ptr(), self.ws.numel(),
                                                 self.stream), "tm_ce_grad_h_bf16")


def _bf16_weight(weight: torch.Tensor) -> torch.Tensor:
    """The contiguous bf16 weight the products run on: ``weight.to(bf16)`` (RNE, as autocast
    casts), or, for an fp32 master whose bf16 working copy is current (attached with
    torchure_amd.attach_bf16_working_params and rewritten by each AdamW step), that copy, which
    holds the same bits, so the cast's read of 4 and write of 2 bytes per element is skipped.
    A copy that does not start on a 16-byte boundary (the optimizer accepts copies at any
    offset) is not taken: this op's kernels read the weight in 16-byte vectors, and the cast
    gives a fresh, aligned buffer with the same bits."""
    if weight.dtype == torch.float32:
        w = current_copy(weight)
        if w is not None and w.data_ptr() % 16 == 0:
            return w.detach()
    return weight.to(torch.bfloat16).contiguous()


def _loss_only(hidden, weight, labels, ignore_index, chunk_size):
    """The loss when no input needs a gradient (e.g. evaluation under torch.no_grad): the
    same logits GEMM and the same per-row arithmetic as the training path, so the same
    bits, without the two gradient GEMMs or the gradient write. The reference's forward
    computes and drops the gradients in this case (fused_linear_ce.py:63-93)."""
    n, v, chunk, mode = _checked(hidden, weight, labels, chunk_size)
    lib = _native.lib()
    stream = _native.stream_handle(hidden.device)
    dt = torch.float32 if mode == "fp32" else torch.bfloat16
    hb = hidden.to(torch.bfloat16) if mode == "autocast" else hidden  # autocast's cast (RNE)
    w = weight.to(dt).contiguous() if mode == "fp32" else _bf16_weight(weight)
    rows_loss = lib.tm_ce_rows_loss_f32 if mode == "fp32" else lib.tm_ce_rows_loss_bf16
    row_loss = torch.empty(n, dtype=torch.float32, device=hidden.device)
    for s in range(0, n, chunk):
        e = min(s + chunk, n)
        logits = _logits(hb[s:e], w, lib, stream) if dt == torch.bfloat16 else _bf16(torch.matmul(hb[s:e], w.t()), dt)
        _native.check(rows_loss(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v, int(ignore_index),
                                row_loss[s:].data_ptr(), stream), "tm_ce_rows_loss")
        del logits
    return _mean_loss(row_loss, labels, n, ignore_index, lib, stream)[0]


def _fp32_forward(ctx, hidden, weight, labels, ignore_index, n, v, chunk):
    """fp32 hidden states outside autocast. The reference then casts the weight to fp32 once
    (fused_linear_ce.py:65), its three products are fp32 GEMMs and its buffers are fp32
    (:66-72). This path does the same: per chunk, fp32 logits from torch.matmul, tm_ce_rows_f32
    in place (the chunk math of :39-51 on fp32 logits), grad_h = grad_logits @ w into the fp32
    grad_hidden (:52,79), and grad_weight += grad_logits^T @ h into a zero-filled fp32 buffer
    (:57,80-81), the reference's own fp32 `+=`. Backward scales both in place."""
    lib = _native.lib()
    stream = _native.stream_handle(hidden.device)
    w = weight.to(torch.float32).contiguous()
    want_h, want_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    grad_hidden = torch.empty(hidden.shape, dtype=torch.float32, device=hidden.device) if want_h else None
    grad_weight = torch.zeros(weight.shape, dtype=torch.float32, device=weight.device) if want_w else None
    row_loss = torch.empty(n, dtype=torch.float32, device=hidden.device)
    for s in range(0, n, chunk):
        e = min(s + chunk, n)
        h = hidden[s:e]
        logits = _bf16(torch.matmul(h, w.t()), torch.float32)  # (C, V) fp32
        _native.check(lib.tm_ce_rows_f32(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v,
                                         int(ignore_index), row_loss[s:].data_ptr(), stream), "tm_ce_rows_f32")
        if want_h:
            torch.matmul(logits, w, out=grad_hidden[s:e])
        if want_w:
            grad_weight += torch.matmul(logits.t(), h)
        del logits
    loss, ctx.n_valid = _mean_loss(row_loss, labels, n, ignore_index, lib, stream)
    ctx.grad_hidden = grad_hidden
    ctx.grad_weight = grad_weight
    ctx.fp32_path = True
    return loss


class _FusedLinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index, chunk_size):
        n, v, chunk, mode = _checked(hidden, weight, labels, chunk_size)
        if mode == "fp32":
            return _fp32_forward(ctx, hidden, weight, labels, ignore_index, n, v, chunk)
        fp32 = mode == "autocast"
        lib = _native.lib()
        stream = _native.stream_handle(hidden.device)
        hb = hidden.to(torch.bfloat16) if fp32 else hidden  # autocast's cast (RNE)
        w = _bf16_weight(weight)  # cast once, not per chunk (or the current working copy)
        want_h, want_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        # bf16 GEMM output either way; for fp32 hidden it is widened and scaled in backward
        grad_hidden = torch.empty(hidden.shape, dtype=torch.bfloat16, device=hidden.device) if want_h else None
        # Chunks' bf16 grad_W wait in `pending` and are folded into the fp32 grad_W several at a
        # time (one pass per fold); the last chunk, and those still pending, wait for backward.
        grad_weight = None
        pending, last_gw = [], None
        accumulated = False
        row_loss = torch.empty(n, dtype=torch.float32, device=hidden.device)
        grad_h_of = GradHidden(w, [min(chunk, n - s) for s in range(0, n, chunk)], lib, stream) if want_h else None
        for s in range(0, n, chunk):
            e = min(s + chunk, n)
            h = hb[s:e]
            logits = _logits(h, w, lib, stream)  # (C, V) bf16
            _native.check(lib.tm_ce_rows_bf16(logits.data_ptr(), v, labels[s:e].data_ptr(), e - s, v,
                                              int(ignore_index), row_loss[s:].data_ptr(), stream),
                          "tm_ce_rows_bf16")
            if want_h:
                grad_h_of(logits, grad_hidden[s:e])
            if want_w:
                gw = _grad_w(logits, h, lib, stream)  # (V, D) bf16
                if e == n:
                    last_gw = gw
                else:
                    pending.append(gw)
                    del gw
                    if len(pending) == FOLD_CHUNKS or len(pending) * pending[0].numel() * 2 >= FOLD_BYTES:
                        if grad_weight is None:
                            grad_weight = torch.empty(weight.shape, dtype=torch.float32, device=weight.device)
                        _fold(lib, grad_weight, pending, accumulated, None, None, stream)
                        accumulated = True
                        pending = []
            del logits
        del grad_h_of
        loss, ctx.n_valid = _mean_loss(row_loss, labels, n, ignore_index, lib, stream)
        ctx.grad_hidden = grad_hidden
        ctx.fp32_hidden = fp32
        ctx.fp32_path = False
        ctx.want_w = want_w
        ctx.grad_weight = grad_weight
        ctx.pending_gw = pending
        ctx.last_gw = last_gw
        ctx.accumulated = accumulated
        ctx.weight_meta = (weight.shape, weight.device)
        return loss

    @staticmethod
    def backward(ctx, grad_out):
        if ctx.n_valid is None:
            raise RuntimeError(
                "fused_linear_cross_entropy: backward called twice. the stashed grads are "
                "consumed in place on the first call, so retain_graph does not work through this op")
        grad_hidden, grad_weight, n_valid = ctx.grad_hidden, ctx.grad_weight, ctx.n_valid
        if ctx.fp32_path:
            ctx.grad_hidden = ctx.grad_weight = ctx.n_valid = None
            # fused_linear_ce.py:107-126: scale = grad_out / n_valid, both buffers scaled in place
            scale = grad_out.detach().to(torch.float32) / n_valid[0]
            if grad_hidden is not None:
                grad_hidden.mul_(scale)
            if grad_weight is not None:
                grad_weight.mul_(scale)
            return grad_hidden, grad_weight, None, None, None
        last_gw, pending = ctx.last_gw, ctx.pending_gw
        ctx.grad_hidden = ctx.grad_weight = ctx.n_valid = ctx.last_gw = ctx.pending_gw = None
        lib = _native.lib()
        stream = _native.stream_handle(n_valid.device)
        g = grad_out.detach().to(torch.float32).contiguous()
        scale_w = None  # an fp32 grad_W that still needs the plain scaling pass
        if ctx.want_w:
            shape, device = ctx.weight_meta
            if last_gw is not None:
                if grad_weight is None:
                    grad_weight = torch.empty(shape, dtype=torch.float32, device=device)
                # the chunks still pending, then the last, with the scaling (at most FOLD_CHUNKS)
                _fold(lib, grad_weight, pending + [last_gw], ctx.accumulated, g, n_valid, stream)
                del last_gw, pending
            else:  # no rows at all: the reference scales its zero-filled buffer
                grad_weight = scale_w = torch.zeros(shape, dtype=torch.float32, device=device)
        if ctx.fp32_hidden and grad_hidden is not None:
            # fp32 hidden: the gradient is fp32 = float(bf16 GEMM result) * scale
            wide = torch.empty(grad_hidden.shape, dtype=torch.float32, device=grad_hidden.device)
            _native.check(lib.tm_ce_widen_scale(wide.data_ptr(), grad_hidden.data_ptr(), grad_hidden.numel(),
                                                g.data_ptr(), n_valid.data_ptr(), stream), "tm_ce_widen_scale")
            grad_hidden, wide = wide, grad_hidden
            del wide
            scale_h = None
        else:
            scale_h = grad_hidden
        rc = lib.tm_ce_scale_grads(
            scale_h.data_ptr() if scale_h is not None else None,
            scale_h.numel() if scale_h is not None else 0,
            scale_w.data_ptr() if scale_w is not None else None,
            scale_w.numel() if scale_w is not None else 0,
            g.data_ptr(), n_valid.data_ptr(), stream)
        _native.check(rc, "tm_ce_scale_grads")
        return grad_hidden, grad_weight, None, None, None


def fused_linear_cross_entropy(
    hidden: torch.Tensor,  # (B, S, D) or (N, D), bf16 or fp32
    weight: torch.Tensor,  # (V, D) lm_head weight
    labels: torch.Tensor,  # (B, S) or (N,), already shifted, int64
    ignore_index: int = -100,
    chunk_size: int | str | None = 1024,
) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.T`` against ``labels`` over the rows whose
    label is not ``ignore_index``, in chunks of ``chunk_size`` rows, as
    torchure/loss/fused_linear_ce.py:130-136 (default 1024 rows, as there: each chunk's bf16
    grad_W is rounded before it is added, so the chunking fixes grad_W's bits).
    ``chunk_size=None`` or ``"auto"`` sizes chunks by a 4 GiB logits budget instead
    (``auto_chunk_rows``): the whole Qwen3 vocabulary for 8K-16K tokens in one chunk, one
    fp32 grad_W pass and large GEMMs, at the cost of other grad_W bits and up to 4 GiB of
    logits plus one bf16 grad_W (V x D) held from forward to backward."""
    if hidden.dim() == 3:
        hidden = hidden.reshape(-1, hidden.shape[-1])
        labels = labels.reshape(-1)
    hidden, labels = hidden.contiguous(), labels.contiguous()
    with CALL_ORDER.call(hidden.device):  # one call's GEMMs at a time per device
        if not (torch.is_grad_enabled() and (hidden.requires_grad or weight.requires_grad)):
            return _loss_only(hidden, weight, labels, ignore_index, chunk_size)
        return _FusedLinearCE.apply(hidden, weight, labels, ignore_index, chunk_size)
