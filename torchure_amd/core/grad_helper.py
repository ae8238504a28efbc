"""Global grad-norm clipping on the gfx950 kernels.

Counterpart of torchure/core/grad_helper.py:8-34 with the same signature,
return value and error behaviour:
  - the pre-clip global L2 norm is returned as a 0-d fp32 device tensor
    (grad_helper.py:34), computed by the deterministic two-pass kernel
    (replaces torch._foreach_norm + stack + vector_norm, grad_helper.py:17-18);
  - clip_coef = clamp(max_norm / (total + 1e-6), max=1.0) stays on device
    (grad_helper.py:32); it is always applied, also when it is 1.0
    (grad_helper.py:33), which is bitwise a no-op;
  - ``max_norm=None`` measures only (grad_helper.py:29-30);
  - no grads at all raises AssertionError (grad_helper.py:15-16).

Deferred clip. When every grad passed in belongs to one torchure_amd AdamW
built with ``defer_clip=True`` (the default), the in-place multiply of
grad_helper.py:33 is not run as a separate pass: the coefficient is handed to
that optimizer, whose next ``step()`` multiplies each grad by it inside the
fused update kernel (the same single fp32 multiply, so for fp32 grads the update
is bitwise the same). For bf16 grads the fused multiply keeps float(g) * coef in
fp32, as the reference trainer does with its fp32 grads (float of the bf16 grads
under autocast); an in-place scale of a bf16 grad has to round the product to
bf16, as torch._foreach_mul_ on a bf16 list does (coefficient rounded too), so
the in-place route steps on those rounded grads. Until that step, ``p.grad``
holds the unscaled values;
``AdamW.materialize_clip()`` applies the pending scale in place if a caller
needs the clipped grads before stepping. A grad modified in place between the
clip and the step makes the step raise (scaling it afterwards would not give
the reference's scale-then-modify result); a grad replaced by a new tensor
steps unscaled, as it does in the reference. In every other case (plain tensors,
params of several optimizers, or ``defer_clip=False``) the grads are scaled in
place immediately by the scale kernel, as the reference does.
"""

from __future__ import annotations

import torch

from torchure_amd import _native
from torchure_amd.core import tables


def grads_of(params) -> tuple[list[torch.Tensor], list[torch.nn.Parameter]]:
    """(grads, holders) for params that carry a grad, in order.

    A master parameter without its own ``.grad`` contributes the bf16 grad of
    its attached working copy (torchure_amd.optimizer.working), if any.
    """
    ps = params if isinstance(params, list) else list(params)
    gs, _ = _native.host().grads(ps, [getattr(p, "_tm_working", None) for p in ps])
    holders = [p for p, g in zip(ps, gs) if g is not None]
    grads = [g for g in gs if g is not None]
    return grads, holders


_NORM_UPLOAD = tables.TableUploader()
_SCALE_UPLOAD = tables.TableUploader()


class NormLaunch:
    """One ``tm_grad_norm`` call with its device tables kept alive; calling it
    enqueues both passes on the device's current stream and writes ``norm``
    (and ``coef`` when clipping)."""

    def __init__(self, grads: list[torch.Tensor], max_norm: float | None,
                 chunk_elems: int = tables.DEFAULT_CHUNK_ELEMS):
        who = "clip_grad_norm"
        device = grads[0].device
        for g in grads:
            if g.device != device:
                raise RuntimeError(f"{who}: all grads must be on one device ({g.device} vs {device})")
        rows = tables.grad_table(grads, who)
        self.device = device
        self.n = len(grads)
        self.chunk_elems = chunk_elems
        self.chunks, self.n_chunks = tables.CHUNKS.get(rows["numel"], chunk_elems, device)
        self.d_rows = _NORM_UPLOAD(rows, device)
        self.ws = torch.empty(_native.workspace_bytes(len(grads)), dtype=torch.uint8, device=device)
        self.norm = torch.empty((), dtype=torch.float32, device=device)
        self.clip = max_norm is not None
        self.max_norm = float(max_norm) if self.clip else 0.0
        self.coef = torch.empty((), dtype=torch.float32, device=device) if self.clip else None
        self.home = torch.cuda.current_stream(device)

    def __call__(self) -> None:
        tables.follow_home_stream(self.home, self.device,
                                  (self.d_rows, self.chunks, self.ws, self.norm, self.coef))
        rc = _native.lib().tm_grad_norm(
            self.d_rows.data_ptr(),
            self.n,
            self.chunks.data_ptr(),
            self.n_chunks,
            self.chunk_elems,
            self.max_norm,
            int(self.clip),
            self.ws.data_ptr(),
            self.norm.data_ptr(),
            self.coef.data_ptr() if self.clip else None,
            _native.stream_handle(self.device),
        )
        _native.check(rc, "tm_grad_norm")


def grad_norm_launch(
    grads: list[torch.Tensor],
    max_norm: float | None,
    chunk_elems: int = tables.DEFAULT_CHUNK_ELEMS,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Launch the two-pass norm over ``grads``; returns (norm, coef-or-None) device scalars."""
    launch = NormLaunch(grads, max_norm, chunk_elems)
    launch()
    return launch.norm, launch.coef


def scale_grads_(
    grads: list[torch.Tensor], coef: torch.Tensor, chunk_elems: int = tables.DEFAULT_CHUNK_ELEMS
) -> None:
    """In-place grads *= coef (the reference's torch._foreach_mul_, grad_helper.py:33)."""
    if not grads:
        return
    who = "clip_grad_norm"
    device = grads[0].device
    rows = tables.grad_table(grads, who)
    chunks, n_chunks = tables.CHUNKS.get(rows["numel"], chunk_elems, device)
    d_rows = _SCALE_UPLOAD(rows, device)
    rc = _native.lib().tm_grad_scale(
        d_rows.data_ptr(),
        len(grads),
        chunks.data_ptr(),
        n_chunks,
        chunk_elems,
        coef.data_ptr(),
        _native.stream_handle(device),
    )
    _native.check(rc, "tm_grad_scale")
    _native.host().bump(grads)


def _check_shard_dims(mesh, shard_dims) -> None:
    """The sharded path (grad_helper.py:20-24) sums the squared norm over each listed mesh
    dimension. A dimension of size 1 makes that sum the identity; larger ones need a
    cross-GPU all_reduce, which this single-GPU build does not provide."""
    for dim in shard_dims:
        size = mesh.size(dim) if mesh is not None else None
        if size != 1:
            raise NotImplementedError(
                f"clip_grad_norm: shard dim {dim!r} has {size} ranks; summing the squared norm "
                "across GPUs needs a collective, and this single-GPU build has none (a mesh "
                "dimension of size 1 is supported)")


def clip_grad_norm(params, mesh, max_norm, shard_dims=()) -> torch.Tensor:
    """Returns the pre-clip global grad norm; clips grads (in place or deferred).

    Signature and semantics of torchure/core/grad_helper.py:8-34. ``mesh`` is
    unused on the local path, as in the reference. ``shard_dims`` may name mesh
    dimensions of size 1, over which the reference's all-reduce of the squared norm
    is the identity; the norm still takes its ``(total ** 2) ** 0.5`` round trip
    (grad_helper.py:20-24), which keeps its bits while the fp32 square neither
    overflows nor underflows, and gives inf above sqrt(FLT_MAX) as the reference does.
    Larger shard dimensions raise NotImplementedError.

    Deferred clip (the default when every grad belongs to one torchure_amd.AdamW whose
    ``defer_clip`` is set): the reference scales ``p.grad`` in place here
    (grad_helper.py:32-33); this function instead hands the coefficient, a device scalar, to
    that optimizer, whose next ``step()`` applies the same fp32 multiply inside the update
    kernel, saving a read and a write of every grad. Until then ``p.grad`` still reads the
    unscaled values. Code that inspects the clipped grads before the step calls
    ``optimizer.materialize_clip()`` (the reference's in-place values) or builds the
    optimizer with ``defer_clip=False``. A grad modified in place before the step makes the
    step raise; a grad replaced by a new tensor steps unscaled, as in the reference.
    """
    if shard_dims:
        _check_shard_dims(mesh, shard_dims)
    grads, holders = grads_of(params)
    if not grads:
        assert grads, "clip_grad_norm got no grads; backward didn't run, or all params are frozen"

    # A clip pending from an earlier call must land before these grads are measured.
    from torchure_amd.optimizer.adamw import materialize_pending_for, owners_of

    owners = owners_of(holders)
    materialize_pending_for(holders, owners)

    from torchure_amd.optimizer.working import cached_norm

    # the last micro-step's fused accumulate+norm may already have measured exactly these grads
    norm = cached_norm(grads)
    coef = None
    if norm is None:
        norm, coef = grad_norm_launch(grads, None if shard_dims else max_norm)
    if shard_dims:
        # grad_helper.py:21-24 with the sum over size-1 dimensions being the identity
        norm = (norm ** 2.0) ** (1.0 / 2.0)
    if max_norm is None:
        return norm
    if coef is None:  # the coefficient of a norm that is already on the device
        coef = torch.empty((), dtype=torch.float32, device=norm.device)
        rc = _native.lib().tm_clip_coef(norm.data_ptr(), float(max_norm), coef.data_ptr(),
                                        _native.stream_handle(norm.device))
        _native.check(rc, "tm_clip_coef")

    opt = next(iter(owners)) if len(owners) == 1 else None
    if opt is not None and opt.defer_clip:
        opt._set_pending_clip(coef, holders, grads)
    else:
        scale_grads_(grads, coef)
    return norm
