"""Pins the CPU oracle before it is trusted (no GPU needed).

- bf16 rounding: bit-exact against torch's own fp32->bf16 cast (golden vectors).
- AdamW recipe: against torch.optim.AdamW(fused=True) on CPU (golden vectors of
  tests/golden/make_golden.py). torch's CPU fused kernel evaluates the moments
  with a different (fp32 lerp-style) formula than its GPU functor, so the pin
  here is a tolerance of a few ulp of the operand scale; the bit-exact pin of the
  GPU recipe is tests/golden/adamw_rocm_*.npz (torch-ROCm's _fused_adamw_).
- closed forms: step-1 update, zero-grad moments, clip known answers, WSD values,
  param-group split counts.
"""

from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest

from oracle import oracle
from tests import _helpers as H
from torchure_amd.workloads import numel, shapes_for

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_bf16_rne_matches_torch_cast():
    """Non-NaN inputs: bit-exact against torch's CPU cast. NaN inputs: torch's CPU
    vector path writes 0xFFFF while its ROCm device path (the one autocast uses on
    the GPU, BFloat16.h:100-114) writes 0x7FC0; the oracle follows the device
    path, and both are NaN. tests/golden/bf16_rne_rocm.npz pins the device bits."""
    z = _load("bf16_rne.npz")
    got = oracle.bf16_rne(z["x"])
    nan = np.isnan(z["x"])
    assert nan.sum() > 2
    assert np.array_equal(got[~nan], z["bits"][~nan])
    assert np.all(got[nan] == 0x7FC0)
    assert np.all(np.isnan(oracle.bf16_to_f32(z["bits"][nan])))


def test_bf16_rne_matches_rocm_cast_if_present():
    path = os.path.join(GOLD, "bf16_rne_rocm.npz")
    if not os.path.exists(path):
        pytest.skip("no torch-ROCm bf16 vectors committed")
    z = np.load(path, allow_pickle=False)
    assert np.array_equal(oracle.bf16_rne(z["x"]), z["bits"])


def test_bf16_rne_planted_truncation_is_caught():
    """A truncating conversion (a plausible bug) disagrees with the golden vectors."""
    z = _load("bf16_rne.npz")
    trunc = (z["x"].view(np.uint32) >> 16).astype(np.uint16)
    assert not np.array_equal(trunc, z["bits"])


CASES = ["adamw_fresh_noclip", "adamw_steady_clip", "adamw_steady_measure"]


def _scaled_err(got, want, scale):
    return np.abs(got.astype(np.float64) - want.astype(np.float64)) / np.spacing(
        np.maximum(scale, np.float32(1e-38)).astype(np.float32)).astype(np.float64)


@pytest.mark.parametrize("case", CASES)
def test_adamw_recipe_vs_torch_cpu_fused(case):
    z = _load(f"{case}.npz")
    shapes = [tuple(int(x) for x in s.strip("()").split(",") if x.strip()) for s in z["shapes"]]
    mn = float(z["max_norm"])
    clip = not math.isnan(mn)
    hy = dict(lr=float(z["lr"]), beta1=float(z["beta1"]), beta2=float(z["beta2"]), eps=float(z["eps"]))
    for k in range(3):
        coef = np.float32(z[f"coef{k}"]) if clip else np.float32(1.0)
        for i, s in enumerate(shapes):
            wd = float(z["weight_decay"]) if len(s) >= 2 else 0.0
            p = z[f"p{k}_{i}"].reshape(-1).copy()
            m = z[f"m{k}_{i}"].reshape(-1).copy()
            v = z[f"v{k}_{i}"].reshape(-1).copy()
            p_prev, m_prev = p.copy(), m.copy()
            g = (z[f"g{k}_{i}"].reshape(-1) * coef).astype(np.float32)
            step_after = float(z["step0"]) + k + 1
            oracle.adamw_update(p, m, v, g, step_after, hy["lr"], hy["beta1"], hy["beta2"], wd, hy["eps"])
            m_scale = np.maximum(np.abs(hy["beta1"] * m_prev), np.abs((1 - hy["beta1"]) * g))
            p_scale = np.maximum(np.abs(p_prev), np.abs(p - p_prev))
            assert _scaled_err(m, z[f"m{k + 1}_{i}"].reshape(-1), m_scale).max() <= 4
            assert H.ulp_diff(v, z[f"v{k + 1}_{i}"].reshape(-1)).max() <= 4
            assert _scaled_err(p, z[f"p{k + 1}_{i}"].reshape(-1), p_scale).max() <= 8
            # bf16 copy of torch's master is RNE of it (equal masters -> equal bf16)
            assert np.array_equal(oracle.bf16_rne(z[f"p{k + 1}_{i}"].reshape(-1)), z[f"bf{k + 1}_{i}"].reshape(-1))
            assert float(z[f"step{k + 1}_{i}"]) == step_after


@pytest.mark.parametrize("case", CASES)
def test_norm_and_coef_vs_torch(case):
    z = _load(f"{case}.npz")
    n = len(z["shapes"])
    mn = float(z["max_norm"])
    for k in range(3):
        grads = [z[f"g{k}_{i}"].reshape(-1) for i in range(n)]
        got = oracle.global_norm(grads)
        want = float(z[f"norm{k}"])
        assert abs(float(got) - want) <= 1e-6 * want
        if not math.isnan(mn):
            # same norm in -> bit-identical coefficient out
            assert oracle.clip_coef(z[f"norm{k}"], mn) == z[f"coef{k}"]


def test_rocm_golden_if_present():
    """Bit-level pin of the GPU recipe: vectors written by torch-ROCm's
    torch._fused_adamw_ on an MI355X (tests/golden/make_golden_gpu.py)."""
    files = sorted(glob.glob(os.path.join(GOLD, "adamw_rocm_*.npz")))
    if not files:
        pytest.skip("no torch-ROCm golden vectors committed")
    for f in files:
        z = np.load(f, allow_pickle=False)
        for case in range(int(z["n_cases"])):
            p = z[f"p_in{case}"].copy()
            m = z[f"m_in{case}"].copy()
            v = z[f"v_in{case}"].copy()
            g = z[f"g{case}"]
            oracle.adamw_update(p, m, v, g, float(z[f"step_after{case}"]), float(z["lr"]), float(z["beta1"]),
                                float(z["beta2"]), float(z[f"wd{case}"]), float(z["eps"]))
            assert H.ulp_diff(p, z[f"p_out{case}"]).max() == 0, (f, case)
            assert H.ulp_diff(m, z[f"m_out{case}"]).max() == 0, (f, case)
            assert H.ulp_diff(v, z[f"v_out{case}"]).max() == 0, (f, case)


def test_step1_closed_form():
    """From m = v = 0 at step 1: m = (1-b1) g, v = (1-b2) g^2 and the update is
    lr * g / (|g| + eps) after decoupled decay (to fp32 rounding)."""
    r = H.rng(3)
    n = 5000
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    lr, b1, b2, wd, eps = 3e-4, 0.9, 0.95, 0.1, 1e-8
    p0 = p.copy()
    oracle.adamw_update(p, m, v, g, 1.0, lr, b1, b2, wd, eps)
    gd = g.astype(np.float64)
    np.testing.assert_allclose(m, (1 - b1) * gd, rtol=2 ** -23)
    np.testing.assert_allclose(v, (1 - b2) * gd * gd, rtol=2 ** -22)
    want = p0.astype(np.float64) * (1 - lr * wd) - lr * gd / (np.abs(gd) + eps)
    np.testing.assert_allclose(p, want, rtol=0, atol=8e-9)


def test_zero_grad_moments():
    r = H.rng(4)
    n = 4000
    m = (r.standard_normal(n) * 1e-4).astype(np.float32)
    v = (np.abs(r.standard_normal(n)) * 1e-8).astype(np.float32)
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    m0, v0 = m.copy(), v.copy()
    oracle.adamw_update(p, m, v, np.zeros(n, np.float32), 1001.0, 3e-4, 0.9, 0.95, 0.0, 1e-8)
    assert np.array_equal(m, (0.9 * m0.astype(np.float64)).astype(np.float32))
    assert np.array_equal(v, (0.95 * v0.astype(np.float64)).astype(np.float32))


def test_adamw_scalars_closed_form():
    for step in (1.0, 2.0, 1001.0, 9800.0):
        ss, bc2s = oracle.adamw_scalars(step, 3e-4, 0.9, 0.95)
        bc1 = np.float32(1 - 0.9 ** step)
        assert ss == np.float32(3e-4 / float(bc1))
        assert bc2s == np.float32(math.sqrt(1 - 0.95 ** step))


def test_clip_known_answers():
    """torchure tests/grad_helper.py:105-146,188-204 on the oracle."""
    assert float(oracle.global_norm([np.array([3.0, 4.0], np.float32)])) == 5.0
    c = oracle.clip_coef(5.0, 1.0)
    assert abs(float(c) - 0.2) < 1e-7
    g = (np.array([3.0, 4.0], np.float32) * c).astype(np.float32)
    np.testing.assert_allclose(g, [0.6, 0.8], rtol=1e-5, atol=1e-6)
    for mx in (0.5, 1.0, 2.0, 10.0):
        assert oracle.clip_coef(0.05, mx) == np.float32(1.0)
    assert float(oracle.global_norm([np.array([3.0, 4.0], np.float32),
                                     np.array([12.0, 0.0], np.float32)])) == 13.0
    assert math.isnan(float(oracle.clip_coef(float("nan"), 1.0)))
    # planted mistake: clamping to max_norm instead of 1.0 amplifies below threshold
    assert min(10.0 / (0.05 + 1e-6), 10.0) != float(oracle.clip_coef(0.05, 10.0))


def test_norm_brute_force_small():
    r = H.rng(5)
    gs = [(r.standard_normal(n) * 1e-3).astype(np.float32) for n in (1, 7, 100, 3)]
    want = math.sqrt(math.fsum(float(x) * float(x) for g in gs for x in g))
    assert abs(float(oracle.global_norm(gs)) - want) <= 1e-6 * want
    bits = [oracle.bf16_rne(g) for g in gs]
    want_b = math.fsum(float(x) ** 2 for b in bits for x in oracle.bf16_to_f32(b))
    assert abs(sum(oracle.sumsq(b) for b in bits) - want_b) <= 1e-12 * want_b


def test_wsd_closed_form():
    T, wr, dr = 10000, 0.001, 0.2
    assert oracle.wsd_scale(0, T, wr, dr) == 0.1
    assert oracle.wsd_scale(9, T, wr, dr) == 1.0
    assert oracle.wsd_scale(10, T, wr, dr) == 1.0
    assert oracle.wsd_scale(8000, T, wr, dr) == 1.0
    assert oracle.wsd_scale(9000, T, wr, dr) == 0.5
    assert oracle.wsd_scale(9800, T, wr, dr) == 0.09999999999999998
    assert 3e-4 * oracle.wsd_scale(9800, T, wr, dr) == 2.999999999999999e-05
    assert oracle.wsd_scale(10000, T, wr, dr) == 0
    assert oracle.wsd_scale(12000, T, wr, dr) == 0  # clamped, no lr floor
    assert oracle.wsd_scale(0, 100, 0.0, 0.1) == 1.0  # W = max(1, 0)


@pytest.mark.parametrize("name,dec,nod,dec_el,nod_el", [
    ("tiny", 15, 9, 2621440, 1536),
    ("qwen3-0.6b-ref", 197, 113, 573964288, 65536),
    ("qwen3-0.6b", 197, 113, 595984384, 65536),
    ("qwen3-4b", 253, 145, 4022272000, 196096),
])
def test_param_group_split(name, dec, nod, dec_el, nod_el):
    shapes = shapes_for(name)
    d, n = oracle.split_groups(shapes)
    assert (len(d), len(n)) == (dec, nod)
    assert sum(numel(shapes[i]) for i in d) == dec_el
    assert sum(numel(shapes[i]) for i in n) == nod_el


def test_bf16_update_equals_widened_update():
    """adamw_update_bf16 (bf16 grad bits, fused clip multiply and bf16 refresh) equals
    adamw_update on the widened, coefficient-scaled fp32 grads."""
    r = H.rng(8)
    n = 3001
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    m = (r.standard_normal(n) * 1e-4).astype(np.float32)
    v = (np.abs(r.standard_normal(n)) * 1e-8).astype(np.float32)
    g = oracle.bf16_rne((r.standard_normal(n) * 1e-3).astype(np.float32))
    coef = np.float32(0.37)
    p2, m2, v2 = p.copy(), m.copy(), v.copy()
    out = np.zeros(n, np.uint16)
    oracle.adamw_update_bf16(p, m, v, g, out, coef, 1, 1001.0, 3e-4, 0.9, 0.95, 0.1, 1e-8)
    gw = (oracle.bf16_to_f32(g) * coef).astype(np.float32)
    oracle.adamw_update(p2, m2, v2, gw, 1001.0, 3e-4, 0.9, 0.95, 0.1, 1e-8)
    assert np.array_equal(p, p2) and np.array_equal(m, m2) and np.array_equal(v, v2)
    assert np.array_equal(out, oracle.bf16_rne(p))


@pytest.mark.parametrize("scale,n", [(1e18, 1000), (3e17, 1000), (1e19, 4), (1e30, 1), (5e18, 13)])
def test_global_norm_overflows_like_torch(scale, n):
    """torch's fp32 norm reductions return inf once the sum of squares leaves the fp32
    range (1000 x 1e18 already does); the oracle follows them, including just below it."""
    import torch

    grads = [np.full(n, scale, dtype=np.float32), np.full(10, 1.0, dtype=np.float32)]
    want = torch.linalg.vector_norm(torch.stack(torch._foreach_norm([torch.from_numpy(g) for g in grads], 2.0)), 2.0)
    got = oracle.global_norm(grads)
    if np.isinf(want.item()):
        assert np.isinf(got)
    else:
        assert abs(float(got) - want.item()) <= 1e-6 * want.item()
