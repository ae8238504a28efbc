"""CPU oracle of the optimizer step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline). The product
package ``torchure_amd`` never imports it; the HIP path has no CPU fallback.

Contents (each restates the cited reference code; the per-element arithmetic
is the C file tm_oracle.c, built by oracle/Makefile):
  bf16_rne / bf16_to_f32  torch/include/torch/headeronly/util/BFloat16.h:100-114
  adamw_update(_bf16)     torch/include/ATen/native/hip/fused_adam_utils.cuh:22-92,106-199
                          + the step increment of torch/optim/adam.py:877
  global_norm             torchure/core/grad_helper.py:17-18 (per-tensor L2 norms,
                          then the L2 norm of the stacked norms)
  clip_coef               torchure/core/grad_helper.py:32 with torch/_tensor.py:1119-1122
  wsd_scale               torchure/optimizer/scheduler.py:17-35
  split_groups            torchure/optimizer/builder.py:37-43
  reference_step          the order of torchure/train/trainer.py:391-397
                          (clip -> AdamW step -> bf16 working copy)
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_BUILD = os.path.join(_HERE, "_build")
_LIBS: dict = {}

_f32p = ctypes.POINTER(ctypes.c_float)


def build() -> None:
    """Compile the C restatement (gcc via oracle/Makefile)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib(threaded: bool = False) -> ctypes.CDLL:
    name = "liborc_mt.so" if threaded else "liborc.so"
    if name in _LIBS:
        return _LIBS[name]
    path = os.path.join(_BUILD, name)
    if not os.path.exists(path):
        build()
    L = ctypes.CDLL(path)
    vp, i64, d, f, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_float, ctypes.c_int
    L.orc_bf16_rne.argtypes = [vp, vp, i64]
    L.orc_bf16_to_f32.argtypes = [vp, vp, i64]
    L.orc_adamw_scalars.argtypes = [f, d, d, d, vp]
    L.orc_adamw_update.argtypes = [vp, vp, vp, vp, i64, f, d, d, d, d, d]
    L.orc_adamw_update_bf16.argtypes = [vp, vp, vp, vp, vp, i64, f, i, f, d, d, d, d, d]
    L.orc_sumsq_f32.argtypes = [vp, i64]
    L.orc_sumsq_f32.restype = d
    L.orc_sumsq_bf16.argtypes = [vp, i64]
    L.orc_sumsq_bf16.restype = d
    L.orc_clip_coef.argtypes = [f, f]
    L.orc_clip_coef.restype = f
    L.orc_num_threads.restype = i
    _LIBS[name] = L
    return L


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


# ------------------------------------------------------------------ bf16


def bf16_rne(x) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round-to-nearest-even, NaN -> 0x7FC0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_rne(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ AdamW


def adamw_scalars(step_after: float, lr: float, beta1: float, beta2: float) -> tuple[float, float]:
    out = np.zeros(2, dtype=np.float32)
    lib().orc_adamw_scalars(float(step_after), lr, beta1, beta2, _ptr(out))
    return float(out[0]), float(out[1])


def adamw_update(p, m, v, g, step_after, lr, beta1, beta2, weight_decay, eps,
                 threaded: bool = False) -> None:
    """In-place AdamW on float32 numpy arrays; ``g`` is the fp32 (clipped) grad.
    ``threaded`` runs the same element-wise code on OpenMP threads (same results)."""
    for a in (p, m, v, g):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    assert p.size == m.size == v.size == g.size
    lib(threaded).orc_adamw_update(_ptr(p), _ptr(m), _ptr(v), _ptr(g), p.size, float(step_after),
                           lr, beta1, beta2, weight_decay, eps)


def adamw_update_bf16(p, m, v, g_bits, out_bits, coef, clip, step_after, lr, beta1, beta2,
                      weight_decay, eps, threaded: bool = False) -> None:
    """In-place AdamW reading bf16 grad bits, fusing the clip multiply and the bf16 refresh."""
    for a in (p, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    assert g_bits.dtype == np.uint16
    assert p.size == m.size == v.size == g_bits.size
    assert out_bits is None or (out_bits.dtype == np.uint16 and out_bits.size == p.size)
    lib(threaded).orc_adamw_update_bf16(
        _ptr(p), _ptr(m), _ptr(v), _ptr(g_bits), _ptr(out_bits) if out_bits is not None else None,
        p.size, float(coef), int(clip), float(step_after), lr, beta1, beta2, weight_decay, eps)


# ------------------------------------------------------------------ clip


def sumsq(g) -> float:
    """Exact-ish fp64 sum of squares of a float32 or bf16-bits array."""
    if g.dtype == np.uint16:
        g = np.ascontiguousarray(g)
        return float(lib().orc_sumsq_bf16(_ptr(g), g.size))
    g = np.ascontiguousarray(g, dtype=np.float32)
    return float(lib().orc_sumsq_f32(_ptr(g), g.size))


# Smallest value that fp32 rounding sends to infinity (2^128 - 2^103).
F32_OVERFLOW = float.fromhex("0x1.ffffffp+127")


def _f32_norm(sq: float) -> np.float32:
    """sqrt of a sum of squares as an fp32 reduction returns it: inf once the sum
    itself would round past FLT_MAX."""
    if sq >= F32_OVERFLOW:
        return np.float32(np.inf)
    return np.float32(np.sqrt(sq))


def global_norm(grads) -> np.float32:
    """grad_helper.py:17-18: per-tensor fp32 L2 norms, then the norm of the stack.

    Each per-tensor norm is computed in fp64 and rounded to fp32 (what a
    well-conditioned fp32 reduction converges to); the outer norm likewise. torch
    reduces both in fp32, so a sum of squares beyond the fp32 range gives inf.
    """
    norms = np.array([_f32_norm(sumsq(g)) for g in grads], dtype=np.float32)
    return _f32_norm(float(np.sum(norms.astype(np.float64) ** 2)))


def clip_coef(total, max_norm) -> np.float32:
    """clamp(max_norm / (total + 1e-6), max=1.0) in fp32, NaN passes through."""
    return np.float32(lib().orc_clip_coef(float(np.float32(total)), float(np.float32(max_norm))))


# ------------------------------------------------------------------ schedule / groups


def wsd_scale(step: int, total_steps: int, warmup_ratio: float, decay_ratio: float) -> float:
    """torchure/optimizer/scheduler.py:17-35, in double."""
    start = total_steps * (1 - decay_ratio)
    warm = max(1, round(total_steps * warmup_ratio))
    if step < warm:
        return (step + 1) / warm
    if step >= start:
        return max(0, 1 - ((step - start) / (decay_ratio * total_steps)))
    return 1.0


def split_groups(shapes) -> tuple[list[int], list[int]]:
    """builder.py:37-43: indices of >=2-D tensors (decay) and of <2-D tensors."""
    dec = [i for i, s in enumerate(shapes) if len(s) >= 2]
    nod = [i for i, s in enumerate(shapes) if len(s) < 2]
    return dec, nod


# ------------------------------------------------------------------ composition


def reference_step(tensors, hyper, max_norm, clip_override=None):
    """One optimizer step of the reference order on numpy state, in place.

    tensors: list of dicts {p, m, v (float32), g (float32 or bf16 bits uint16),
             step (python float, before increment), wd (float), out (uint16 or None)}
    hyper:   dict lr, beta1, beta2, eps
    max_norm: float or None
    clip_override: use this fp32 coefficient instead of the oracle's own
    Returns (norm, coef).
    """
    grads = [t["g"] for t in tensors]
    norm = global_norm(grads)
    coef = np.float32(1.0)
    clip = max_norm is not None
    if clip:
        coef = clip_coef(norm, max_norm) if clip_override is None else np.float32(clip_override)
    for t in tensors:
        step_after = np.float32(np.float32(t["step"]) + np.float32(1.0))
        t["step"] = float(step_after)
        g = t["g"]
        if g.dtype == np.uint16:
            adamw_update_bf16(t["p"], t["m"], t["v"], g, t.get("out"), coef, clip, step_after,
                              hyper["lr"], hyper["beta1"], hyper["beta2"], t["wd"], hyper["eps"])
        else:
            gc = (g * coef).astype(np.float32) if clip else g.astype(np.float32)
            adamw_update(t["p"], t["m"], t["v"], np.ascontiguousarray(gc), step_after,
                         hyper["lr"], hyper["beta1"], hyper["beta2"], t["wd"], hyper["eps"])
            if t.get("out") is not None:
                t["out"][...] = bf16_rne(t["p"])
    return norm, coef
