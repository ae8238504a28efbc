"""GPU parity of the HIP optimizer step against the CPU oracle (and torch-ROCm).

Bar (from the port's contract): bf16 working copies bit-exact given equal fp32
masters; fp32 master / m / v within 2 ulp; grad norm within 1e-6 relative.
Against the oracle, which restates the same rounding sequence, the kernels are
expected to be bit-exact; the tests assert the contract tolerance and record
exactness separately where it is the stronger claim.
"""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import _helpers as H
from torchure_amd.workloads import numel, ragged_shapes, shapes_for

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import torchure_amd

    torchure_amd._native.lib()  # fail loudly if the HIP library is missing
    yield


def _run_step(host, *, max_norm=1.0, grad_on_master=False):
    import torchure_amd as ta

    params, work, opt = H.device_setup(host, DEV, grad_on_master=grad_on_master)
    norm = ta.clip_grad_norm(params, None, max_norm)
    coef = opt._pending[0].clone() if opt._pending is not None else None
    opt.step()
    torch.cuda.synchronize()
    return params, work, opt, norm, coef


def test_tiny_config_step_matches_oracle():
    """The tiny Qwen3-style set (fresh state, clip triggers at norm ~1.62)."""
    host = H.make_host_set(shapes_for("tiny"), seed=1, steady=False)
    params, work, opt, norm, coef = _run_step(host)
    tens = H.oracle_tensors(host)
    ref_norm, _ = oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
    assert abs(float(norm.item()) - float(ref_norm)) <= 1e-6 * float(ref_norm)
    assert float(coef.item()) == float(oracle.clip_coef(norm.item(), 1.0))
    assert float(coef.item()) < 1.0  # the clip triggered
    w = H.compare_state(params, work, opt, tens)
    assert w["p"] <= 2 and w["m"] <= 2 and w["v"] <= 2, w
    assert w["bf16"] == 0 and w["step"] == 0, w
    # stronger than the contract: same rounding sequence -> bit-exact
    assert w["p"] == 0 and w["m"] == 0 and w["v"] == 0, w


def test_bf16_copy_is_rne_of_master():
    host = H.make_host_set(shapes_for("tiny")[:6], seed=2)
    params, work, opt, _, _ = _run_step(host)
    for p, w in zip(params, work):
        assert np.array_equal(H.from_dev_bf16(w), oracle.bf16_rne(p.detach().cpu().numpy().reshape(-1)))


def test_attach_and_refresh_cast_is_rne():
    """attach_bf16_working_params and refresh_bf16_working_params write RNE(master)
    (torch/headeronly/util/BFloat16.h:100-114, NaN -> 0x7FC0) bit for bit: special values,
    halfway cases, odd lengths, and masters that are views at offsets that are not 16-byte
    aligned (the element-wise path)."""
    import torchure_amd as ta

    r = H.rng(91)
    base = (r.standard_normal(300_000) * 10.0).astype(np.float32)
    base[:12] = [np.nan, np.inf, -np.inf, -0.0, 1e-40, -1e-42, 3.4e38, 1.0 + 2.0 ** -8,
                 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 65504.0, 2.0 ** -126]
    dev = torch.from_numpy(base).to(DEV)
    spans = [(0, 12), (12, 12 + 8 * 1000), (9000, 9000 + 16384 * 3 + 5), (100_001, 100_001 + 777),
             (200_003, 200_003 + 40_000)]
    params = [torch.nn.Parameter(dev[a:b]) for a, b in spans]
    work = ta.attach_bf16_working_params(params)
    torch.cuda.synchronize()
    for (a, b), w in zip(spans, work):
        assert np.array_equal(H.from_dev_bf16(w), oracle.bf16_rne(base[a:b])), (a, b)
    with torch.no_grad():
        for p in params:
            p.mul_(-0.5)
    ta.refresh_bf16_working_params(params)
    torch.cuda.synchronize()
    for p, w in zip(params, work):
        assert np.array_equal(H.from_dev_bf16(w), oracle.bf16_rne(p.detach().cpu().numpy().reshape(-1)))


def test_norm_vs_fp64_and_deterministic():
    import torchure_amd as ta
    from torchure_amd.core.grad_helper import grad_norm_launch

    host = H.make_host_set(shapes_for("tiny"), seed=3, grad_std=2e-3)
    params, work, opt = H.device_setup(host, DEV)
    grads = [w.grad for w in work]
    n1, c1 = grad_norm_launch(grads, 1.0)
    n2, c2 = grad_norm_launch(grads, 1.0)
    torch.cuda.synchronize()
    exact = np.sqrt(sum(oracle.sumsq(h["g"]) for h in host))
    assert abs(float(n1.item()) - exact) <= 1e-6 * exact
    # bitwise identical on a second run (no atomics in the result path)
    assert n1.view(torch.int32).item() == n2.view(torch.int32).item()
    assert c1.view(torch.int32).item() == c2.view(torch.int32).item()
    assert float(c1.item()) == float(oracle.clip_coef(n1.item(), 1.0))
    # the package entry point reports the same pre-clip norm
    n3 = ta.clip_grad_norm(params, None, None)
    assert n3.view(torch.int32).item() == n1.view(torch.int32).item()


def test_steady_state_no_clip_config2():
    """The steady state (step 1000 -> 1001, m ~ N(0,1e-4), v = |N|*1e-8) with grads rescaled
    so the global norm is 0.5 and the clip does not trigger (coef exactly 1)."""
    shapes = shapes_for("tiny")
    host = H.make_host_set(shapes, seed=4)
    total = np.sqrt(sum(oracle.sumsq(h["g"]) for h in host))
    for h in host:
        h["g"] = oracle.bf16_rne(oracle.bf16_to_f32(h["g"]) * np.float32(0.5 / total))
    params, work, opt, norm, coef = _run_step(host)
    assert float(norm.item()) < 1.0 and float(coef.item()) == 1.0
    tens = H.oracle_tensors(host)
    oracle.reference_step(tens, H.HYPER, 1.0)
    w = H.compare_state(params, work, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w


def test_ragged_three_chained_steps():
    """The ragged list in miniature: odd lengths (scalar tail), 1-D no-decay tensors,
    all-zero grads, three chained steps with drift checked every step."""
    shapes = ragged_shapes(n_tensors=300, max_log2=16, seed=9)
    host = H.make_host_set(shapes, seed=5, zero_grad_every=100)
    params, work, opt = H.device_setup(host, DEV)
    tens = H.oracle_tensors(host)
    import torchure_amd as ta

    r = H.rng(55)
    for k in range(3):
        if k:
            for i, h in enumerate(host):
                g = (r.standard_normal(h["p"].size) * 1e-3).astype(np.float32)
                if i % 100 == 99:
                    g[:] = 0
                h["g"] = oracle.bf16_rne(g)
                tens[i]["g"] = h["g"]
                work[i].grad = H.to_dev_bf16(h["g"], h["shape"], DEV)
        norm = ta.clip_grad_norm(params, None, 1.0)
        coef = opt._pending[0].clone()
        opt.step()
        torch.cuda.synchronize()
        ref_norm, _ = oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
        assert abs(float(norm.item()) - float(ref_norm)) <= 1e-6 * float(ref_norm)
        w = H.compare_state(params, work, opt, tens)
        assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, (k, w)


def test_fp32_accumulated_grads_config3():
    """Grad accumulation in miniature: 4 bf16 micro-grads summed into fp32 buffers by the
    accumulate kernel, scaled to global norm 5 (clip coef ~0.2), WSD lr at the
    decay-phase step 9800 of T=10000 (lr = 3e-4 * 0.1)."""
    import torchure_amd as ta
    from torchure_amd.optimizer.working import accumulate_grad_

    shapes = shapes_for("tiny")
    host = H.make_host_set(shapes, seed=6, grad_dtype="f32")
    r = H.rng(66)
    micro = [[oracle.bf16_rne((r.standard_normal(numel(s)) * 2e-3).astype(np.float32)) for s in shapes]
             for _ in range(4)]
    acc_ref = [np.zeros(numel(s), np.float32) for s in shapes]
    for k in range(4):
        for i in range(len(shapes)):
            acc_ref[i] = (acc_ref[i] + oracle.bf16_to_f32(micro[k][i])).astype(np.float32)
    total = np.sqrt(sum(oracle.sumsq(a) for a in acc_ref))
    scale = np.float32(5.0 / total)
    # the scaled micro-grads are what the device accumulates
    micro = [[oracle.bf16_rne(oracle.bf16_to_f32(mg) * scale) for mg in mk] for mk in micro]
    acc_ref = [np.zeros(numel(s), np.float32) for s in shapes]
    for k in range(4):
        for i in range(len(shapes)):
            acc_ref[i] = (acc_ref[i] + oracle.bf16_to_f32(micro[k][i])).astype(np.float32)
    for i, h in enumerate(host):
        h["g"] = acc_ref[i]
    params, work, opt = H.device_setup(host, DEV, grad_on_master=True)
    for p in params:
        p.grad.zero_()
    for k in range(4):
        for i, p in enumerate(params):
            accumulate_grad_(p.grad, H.to_dev_bf16(micro[k][i], p.shape, DEV))
    for i, p in enumerate(params):
        assert np.array_equal(p.grad.cpu().numpy().reshape(-1), acc_ref[i])
    sched = ta.build_scheduler(opt, {"type": "wsd", "total_steps": 10000, "warmup_ratio": 0.001,
                                     "decay_ratio": 0.2})
    sched.last_epoch = 9799
    sched.step()  # -> last_epoch 9800, the lr the step at index 9800 uses
    lr = opt.param_groups[0]["lr"]
    assert lr == 3e-4 * oracle.wsd_scale(9800, 10000, 0.001, 0.2)
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    assert abs(float(norm.item()) - 5.0) < 1e-2 and float(coef.item()) < 0.21
    tens = H.oracle_tensors(host)
    ref_norm, _ = oracle.reference_step(tens, dict(H.HYPER, lr=lr), 1.0, clip_override=float(coef.item()))
    assert abs(float(norm.item()) - float(ref_norm)) <= 1e-6 * float(ref_norm)
    w = H.compare_state(params, work, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w


def test_matches_torch_rocm_fused_adamw():
    """Same inputs through torch.optim.AdamW(fused=True) on the GPU (the reference's
    optimizer, fed fp32 grads = widened bf16, clipped by the reference composition)."""
    import torchure_amd as ta

    shapes = shapes_for("tiny")
    host = H.make_host_set(shapes, seed=7)
    params, work, opt, norm, coef = _run_step(host)
    ref = [torch.nn.Parameter(torch.from_numpy(h["p"].copy()).view(h["shape"]).to(DEV)) for h in host]
    groups = [{"params": [p for p in ref if p.dim() >= 2], "weight_decay": H.WD},
              {"params": [p for p in ref if p.dim() < 2], "weight_decay": 0.0}]
    topt = torch.optim.AdamW(groups, lr=H.HYPER["lr"], betas=(H.HYPER["beta1"], H.HYPER["beta2"]),
                             eps=H.HYPER["eps"], fused=True)
    for p, h in zip(ref, host):
        p.grad = torch.from_numpy(oracle.bf16_to_f32(h["g"]).copy()).view(h["shape"]).to(DEV)
        topt.state[p]["step"] = torch.tensor(h["step"], dtype=torch.float32, device=DEV)
        topt.state[p]["exp_avg"] = torch.from_numpy(h["m"].copy()).view(h["shape"]).to(DEV)
        topt.state[p]["exp_avg_sq"] = torch.from_numpy(h["v"].copy()).view(h["shape"]).to(DEV)
    grads = [p.grad for p in ref]
    total = torch.linalg.vector_norm(torch.stack(torch._foreach_norm(grads, 2.0)), 2.0)
    assert abs(total.item() - norm.item()) <= 1e-6 * total.item()
    torch._foreach_mul_(grads, coef)  # same coefficient: isolates the update kernel
    topt.step()
    torch.cuda.synchronize()
    worst = {"p": 0, "m": 0, "v": 0}
    exact = 0
    total_n = 0
    for p, q in zip(params, ref):
        a, b = opt.state[p], topt.state[q]
        dp = H.ulp_diff(p.detach().cpu().numpy().reshape(-1), q.detach().cpu().numpy().reshape(-1))
        worst["p"] = max(worst["p"], int(dp.max()))
        worst["m"] = max(worst["m"], int(H.ulp_diff(a["exp_avg"].cpu().numpy().reshape(-1),
                                                    b["exp_avg"].cpu().numpy().reshape(-1)).max()))
        worst["v"] = max(worst["v"], int(H.ulp_diff(a["exp_avg_sq"].cpu().numpy().reshape(-1),
                                                    b["exp_avg_sq"].cpu().numpy().reshape(-1)).max()))
        exact += int((dp == 0).sum())
        total_n += dp.size
        assert a["step"].item() == b["step"].item()
    print(f"vs torch-ROCm fused AdamW: max ulp {worst}, master bit-exact {exact}/{total_n}")
    assert worst["p"] <= 2 and worst["m"] <= 2 and worst["v"] <= 2, worst
    # bf16 working copies equal torch's bf16 cast of the same master
    for p, w in zip(params, work):
        assert torch.equal(w, p.detach().to(torch.bfloat16))


_CORNERS = {
    # name: (lr, beta1, beta2, weight_decay, eps, step, p scale, m scale, v scale, g scale)
    "lr_zero": (0.0, 0.9, 0.95, 0.1, 1e-8, 10.0, 0.02, 1e-4, 1e-8, 1e-3),
    "betas_zero": (1e-3, 0.0, 0.0, 0.1, 1e-8, 10.0, 0.02, 1e-4, 1e-8, 1e-3),
    "strong_decay": (1e-2, 0.9, 0.95, 1.0, 1e-8, 10.0, 0.02, 1e-4, 1e-8, 1e-3),
    "large_eps": (1e-3, 0.9, 0.95, 0.1, 1.0, 10.0, 0.02, 1e-4, 1e-8, 1e-3),
    "step_1e6": (3e-4, 0.9, 0.95, 0.1, 1e-8, 1e6, 0.02, 1e-4, 1e-8, 1e-3),
    "fresh": (3e-4, 0.9, 0.999, 0.1, 1e-8, 0.0, 0.02, 0.0, 0.0, 1e-3),
    "tiny_values": (3e-4, 0.9, 0.95, 0.1, 1e-8, 100.0, 1e-30, 1e-39, 1e-44, 1e-30),
    "huge_grads": (3e-4, 0.9, 0.95, 0.1, 1e-8, 100.0, 1.0, 1e15, 1e30, 1e20),
    "zero_grads": (3e-4, 0.9, 0.95, 0.1, 1e-8, 100.0, 0.02, 1e-4, 1e-8, 0.0),
    "half_betas": (1e-3, 0.5, 0.5, 0.0, 1e-12, 3.0, 0.02, 1e-4, 1e-8, 1e-3),
}


@pytest.mark.parametrize("case", sorted(_CORNERS))
def test_hyperparameter_corners_match_torch_rocm(case):
    """Corner regimes of the update (zero lr or betas, strong decay, large eps, very late and
    fresh steps, values near the fp32 range limits, zero grads) against torch-ROCm's
    AdamW(fused=True) on the same device, fp32 grads: within the 2-ulp contract, bit-exact
    in practice."""
    import torchure_amd as ta

    lr, b1, b2, wd, eps, step, ps_, ms_, vs_, gs_ = _CORNERS[case]
    g = torch.Generator(device=DEV).manual_seed(sum(map(ord, case)))  # stable across runs
    shapes = [(64, 64), (1000,), (7,)]
    init = [(torch.randn(sh, device=DEV, generator=g) * ps_,
             torch.randn(sh, device=DEV, generator=g) * ms_,
             torch.randn(sh, device=DEV, generator=g).abs() * vs_,
             torch.randn(sh, device=DEV, generator=g) * gs_) for sh in shapes]
    mine = [torch.nn.Parameter(t[0].clone()) for t in init]
    ref = [torch.nn.Parameter(t[0].clone()) for t in init]
    opt = ta.AdamW(mine, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, fused=True)
    topt = torch.optim.AdamW(ref, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, fused=True)
    for o, ps in ((opt, mine), (topt, ref)):
        for q, t in zip(ps, init):
            q.grad = t[3].clone()
            o.state[q]["step"] = torch.tensor(step, dtype=torch.float32, device=DEV)
            o.state[q]["exp_avg"] = t[1].clone()
            o.state[q]["exp_avg_sq"] = t[2].clone()
    opt.step()
    topt.step()
    torch.cuda.synchronize()
    worst, exact, n = 0, 0, 0
    for a, b in zip(mine, ref):
        pairs = [(a, b)] + [(opt.state[a][k], topt.state[b][k]) for k in ("exp_avg", "exp_avg_sq", "step")]
        for x, y in pairs:
            d = H.ulp_diff(x.detach().cpu().numpy().reshape(-1), y.detach().cpu().numpy().reshape(-1))
            worst = max(worst, int(d.max()))
            exact += int((d == 0).sum())
            n += d.size
    print(f"{case}: max ulp {worst}, bit-exact {exact}/{n}")
    assert worst <= 2, (case, worst)


@pytest.mark.parametrize("grad_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("scale", [1e18, 3e17])
def test_norm_overflow_matches_torch(grad_dtype, scale):
    """torch's fp32 norm reductions give inf once the sum of squares leaves the fp32 range
    (1000 x 1e18 does; 1000 x 3e17 does not), and the clip coefficient becomes 0. The fp64
    norm is cut at the same point, so the clipped step matches the reference's: norm bit for
    bit when finite within 1e-6, and the update equal to torch's fused AdamW on the grads
    torch's clip composition leaves."""
    import torchure_amd as ta
    from oracle.torch_composition import clip_grad_norm_reference

    shapes = [(1000,), (10,)]
    vals = [scale, 1.0]
    mine = [torch.nn.Parameter(torch.full(sh, 0.01, device=DEV)) for sh in shapes]
    ref = [torch.nn.Parameter(torch.full(sh, 0.01, device=DEV)) for sh in shapes]
    if grad_dtype == "bf16":
        work = ta.attach_bf16_working_params(mine)
        for w, sh, v in zip(work, shapes, vals):
            w.grad = torch.full(sh, v, device=DEV, dtype=torch.bfloat16)
        gvals = [float(torch.tensor(v, dtype=torch.bfloat16)) for v in vals]
    else:
        for p, sh, v in zip(mine, shapes, vals):
            p.grad = torch.full(sh, v, device=DEV)
        gvals = vals
    for q, sh, v in zip(ref, shapes, gvals):
        q.grad = torch.full(sh, v, device=DEV)
    opt = ta.AdamW(mine, lr=1e-3, fused=True)
    topt = torch.optim.AdamW(ref, lr=1e-3, fused=True)
    norm = ta.clip_grad_norm(mine, None, 1.0)
    want = clip_grad_norm_reference([q.grad for q in ref], 1.0)
    torch.cuda.synchronize()
    if math.isinf(want.item()):
        assert math.isinf(norm.item())
    else:
        assert abs(norm.item() - want.item()) <= 1e-6 * want.item()
    opt.step()
    topt.step()
    torch.cuda.synchronize()
    if math.isinf(want.item()):  # coefficient 0: the reference steps on zeroed grads
        for a, b in zip(mine, ref):
            assert torch.equal(a, b)
            assert torch.equal(opt.state[a]["exp_avg"], topt.state[b]["exp_avg"])


def test_reference_clip_known_answers():
    """torchure tests/grad_helper.py:105-160,188-204 restated on the GPU path."""
    import torchure_amd as ta

    def params_with(grads):
        out = []
        for g in grads:
            p = torch.nn.Parameter(torch.zeros_like(g, device=DEV))
            p.grad = g.to(DEV).clone()
            out.append(p)
        return out

    # below threshold: bitwise untouched for every max_norm
    for mx in (0.5, 1.0, 2.0, 10.0):
        ps = params_with([torch.tensor([0.03, 0.04]), torch.zeros(3)])
        before = [p.grad.clone() for p in ps]
        total = ta.clip_grad_norm(ps, None, mx)
        torch.testing.assert_close(total.cpu(), torch.tensor(0.05), rtol=1e-5, atol=1e-8)
        for p, b in zip(ps, before):
            assert torch.equal(p.grad, b)
    # [3,4] -> 5, clipped to [0.6, 0.8]
    ps = params_with([torch.tensor([3.0, 4.0])])
    total = ta.clip_grad_norm(ps, None, 1.0)
    assert total.item() == 5.0
    torch.testing.assert_close(ps[0].grad.cpu(), torch.tensor([0.6, 0.8]), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(torch.linalg.vector_norm(ps[0].grad).cpu(), torch.tensor(1.0),
                               rtol=1e-5, atol=1e-6)
    # None measures only
    ps = params_with([torch.tensor([3.0, 4.0])])
    before = ps[0].grad.clone()
    assert ta.clip_grad_norm(ps, None, None).item() == 5.0
    assert torch.equal(ps[0].grad, before)
    # no grads asserts
    with pytest.raises(AssertionError):
        ta.clip_grad_norm([torch.nn.Parameter(torch.zeros(4, device=DEV))], None, 1.0)
    # replicated grads are not reduced: 13.0
    ps = params_with([torch.tensor([3.0, 4.0]), torch.tensor([12.0, 0.0])])
    assert ta.clip_grad_norm(ps, None, 100.0).item() == 13.0
    # bf16 grads scaled in place are rounded RNE, as torch._foreach_mul_ on bf16 does
    g = torch.randn(1000, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    ps = params_with([g])
    ref = g.clone().to(DEV)
    total = ta.clip_grad_norm(ps, None, 1.0)
    rn = torch.linalg.vector_norm(ref.float())
    torch._foreach_mul_([ref], torch.clamp(1.0 / (rn + 1e-6), max=1.0))
    assert abs(total.item() - rn.item()) <= 1e-6 * rn.item()
    assert torch.equal(ps[0].grad, ref)


def test_shard_dims_of_size_one():
    """clip_grad_norm with shard_dims naming mesh dimensions of size 1. The reference's sharded
    path (torchure/core/grad_helper.py:20-24) squares the norm, sums it over each dimension
    (the identity for one rank) and takes the root. Checked: the sharded case of
    tests/grad_helper.py:163-185 at one rank; bitwise equality with the local path for an
    ordinary norm (eager and deferred clip); inf, and a zero coefficient, once the fp32 square
    overflows, as torch's ops give."""
    import torchure_amd as ta

    class Mesh:
        def size(self, dim):
            return 1

    def params_with(grads):
        out = []
        for g in grads:
            p = torch.nn.Parameter(torch.zeros_like(g, device=DEV))
            p.grad = g.to(DEV).clone()
            out.append(p)
        return out

    full = torch.arange(1, 5, dtype=torch.float32)
    true = full.norm()
    mx = (true / 2).item()
    ps = params_with([full])
    total = ta.clip_grad_norm(ps, Mesh(), mx, shard_dims=("dp",))
    torch.testing.assert_close(total.cpu(), true, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ps[0].grad.cpu(), full * (mx / true), rtol=1e-5, atol=1e-6)

    gen = torch.Generator().manual_seed(5)
    grads = [torch.randn(1000, generator=gen) * 3e-3, torch.randn(37, 11, generator=gen)]
    a, b = params_with(grads), params_with(grads)
    na = ta.clip_grad_norm(a, None, 1.0)
    nb = ta.clip_grad_norm(b, Mesh(), 1.0, shard_dims=("dp", "tp"))
    assert na.view(torch.int32).item() == nb.view(torch.int32).item()
    for pa, pb in zip(a, b):
        assert torch.equal(pa.grad, pb.grad)
    # the same through an optimizer that defers the clip into its step
    a, b = params_with(grads), params_with(grads)
    opt_a = ta.build_optimizer(torch.nn.ParameterList(a), "adamw", {"lr": 1e-3, "fused": True})
    opt_b = ta.build_optimizer(torch.nn.ParameterList(b), "adamw", {"lr": 1e-3, "fused": True})
    ta.clip_grad_norm(a, None, 1.0)
    ta.clip_grad_norm(b, Mesh(), 1.0, shard_dims=("dp",))
    opt_a.step()
    opt_b.step()
    for pa, pb in zip(a, b):
        assert torch.equal(pa, pb)

    big = torch.tensor([1e20, 0.0, -3.0])
    ps = params_with([big])
    total = ta.clip_grad_norm(ps, Mesh(), 1.0, shard_dims=("dp",))
    ref_total = (torch.linalg.vector_norm(big.to(DEV)) ** 2.0) ** 0.5
    ref_coef = torch.clamp(1.0 / (ref_total + 1e-6), max=1.0)
    assert math.isinf(total.item()) and math.isinf(ref_total.item())
    assert torch.equal(ps[0].grad, big.to(DEV) * ref_coef)


def test_skip_params_without_grad_and_zero_numel():
    import torchure_amd as ta

    host = H.make_host_set([(64, 8), (16,), (0,), (40,)], seed=8)
    params, work, opt = H.device_setup(host, DEV)
    work[1].grad = None  # this param has no grad: skipped, step stays
    ta.clip_grad_norm(params, None, 1.0)
    opt.step()
    torch.cuda.synchronize()
    assert opt.state[params[1]]["step"].item() == host[1]["step"]
    assert np.array_equal(params[1].detach().cpu().numpy().reshape(-1), host[1]["p"])
    assert opt.state[params[2]]["step"].item() == host[2]["step"] + 1  # empty tensor still steps
    assert opt.state[params[0]]["step"].item() == host[0]["step"] + 1


def test_unaligned_views_use_scalar_path():
    """Tensors that start at odd element offsets (not 16-byte aligned) and have
    odd lengths go through the element-wise path and must match the oracle."""
    import torchure_amd as ta

    sizes = [37, 1000, 4099, 1]
    host = H.make_host_set([(n,) for n in sizes], seed=10)
    flat_p = torch.zeros(sum(sizes) + 8, device=DEV)
    params = []
    off = 1
    for h, n in zip(host, sizes):
        view = flat_p[off:off + n]
        view.copy_(torch.from_numpy(h["p"]))
        p = view.detach().requires_grad_(True)
        p.grad = torch.from_numpy(oracle.bf16_to_f32(h["g"]).copy()).to(DEV)
        params.append(p)
        off += n
    opt = ta.AdamW(params, lr=H.HYPER["lr"], betas=(H.HYPER["beta1"], H.HYPER["beta2"]),
                   weight_decay=H.WD, fused=True)
    for p, h in zip(params, host):
        opt.state[p]["step"] = torch.tensor(h["step"], dtype=torch.float32, device=DEV)
        opt.state[p]["exp_avg"] = torch.from_numpy(h["m"].copy()).to(DEV)
        opt.state[p]["exp_avg_sq"] = torch.from_numpy(h["v"].copy()).to(DEV)
        h["wd"] = H.WD
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    tens = H.oracle_tensors(host)
    for t, h in zip(tens, host):
        t["g"] = oracle.bf16_to_f32(h["g"]).copy()
        t["out"] = None
    oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
    w = H.compare_state(params, None, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w


def test_state_dict_roundtrip_with_torch_adamw():
    """optimizer.state_dict() loads into torch.optim.AdamW and back (the layout
    torchure/checkpoint/checkpointer.py:43-60 saves), and training continues identically."""
    import torchure_amd as ta

    host = H.make_host_set(shapes_for("tiny")[:8], seed=12)
    params, work, opt, _, _ = _run_step(host)
    sd = opt.state_dict()
    ref = [torch.nn.Parameter(p.detach().clone()) for p in params]
    groups = [{"params": [p for p in ref if p.dim() >= 2], "weight_decay": H.WD},
              {"params": [p for p in ref if p.dim() < 2], "weight_decay": 0.0}]
    topt = torch.optim.AdamW(groups, lr=H.HYPER["lr"], betas=(H.HYPER["beta1"], H.HYPER["beta2"]),
                             fused=True)
    topt.load_state_dict(sd)
    tsd = topt.state_dict()
    assert tsd["param_groups"] == sd["param_groups"]
    assert set(sd["state"]) == set(tsd["state"])
    for k in sd["state"]:
        for key in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(sd["state"][k][key], tsd["state"][k][key])
            assert sd["state"][k][key].dtype == torch.float32
    # and back: a fresh torchure_amd AdamW loads torch's dict
    opt2 = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                              {"lr": H.HYPER["lr"], "weight_decay": H.WD,
                               "betas": (H.HYPER["beta1"], H.HYPER["beta2"]), "fused": True})
    opt2.load_state_dict(tsd)
    for p in params:
        for key in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(opt2.state[p][key], opt.state[p][key])
        assert opt2.state[p]["step"].device == p.device


@pytest.mark.parametrize("config", ["qwen3-0.6b", "qwen3-0.6b-ref", "qwen3-4b"])
def test_full_size_properties(config):
    """Configs 2 and 4 at full size (596M / 4.02B params, and the reference's default 0.6B
    shape with MLP 2816, 574M): norm vs fp64 over every grad, the bf16 copy is RNE(master)
    everywhere, and sampled tensors -- including the tied embedding, the largest tensor --
    match the oracle bit for bit."""
    import torchure_amd as ta

    shapes = shapes_for(config)
    g = torch.Generator(device=DEV).manual_seed(0)
    params, grads = [], []
    for s in shapes:
        p = torch.nn.Parameter(torch.randn(s, device=DEV, generator=g) * 0.02)
        params.append(p)
    work = ta.attach_bf16_working_params(params)
    for w in work:
        w.grad = (torch.randn(w.shape, device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
        grads.append(w.grad)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})
    sample = [0, 1, 5, 6, 200, len(shapes) - 1]
    before = {i: (params[i].detach().cpu().numpy().reshape(-1).copy(),
                  H.from_dev_bf16(grads[i]).copy()) for i in sample}
    exact_sq = 0.0
    for gr in grads:
        exact_sq += float(torch.sum(gr.double() ** 2).item())
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    assert abs(norm.item() - np.sqrt(exact_sq)) <= 1e-6 * np.sqrt(exact_sq)
    for p, w in zip(params, work):
        assert torch.equal(w, p.detach().to(torch.bfloat16))
    for i in sample:
        p0, gb = before[i]
        n = p0.size
        t = [dict(p=p0.copy(), m=np.zeros(n, np.float32), v=np.zeros(n, np.float32), g=gb, step=0.0,
                  wd=0.1 if len(shapes[i]) >= 2 else 0.0, out=np.zeros(n, np.uint16))]
        oracle.adamw_update_bf16(t[0]["p"], t[0]["m"], t[0]["v"], gb, t[0]["out"], float(coef.item()), 1,
                                 1.0, 3e-4, 0.9, 0.95, t[0]["wd"], 1e-8, threaded=True)
        got = params[i].detach().cpu().numpy().reshape(-1)
        assert int(H.ulp_diff(got, t[0]["p"]).max()) == 0, i
        assert np.array_equal(opt.state[params[i]]["exp_avg"].cpu().numpy().reshape(-1), t[0]["m"])


@pytest.mark.parametrize("config", ["qwen3-0.6b", "qwen3-4b"])
def test_full_size_steady_state(config):
    """The Qwen3-0.6B and Qwen3-4B parameter sets at full size, from the steady state the
    reference step runs in (torchure/train/trainer.py:391-397): state['step'] 1000 (the kernel
    uses t = 1001), m ~ N(0, 1e-4), v = |N(0,1)| * 1e-8, masters ~ N(0, 0.02). The 0.6B set
    rescales its bf16 grads to global norm 0.5, so clip 1.0 does not trigger (the coefficient is
    exactly 1.0); the 4B set keeps N(0, 1e-3) grads, whose norm (~63) does trigger it. The norm is checked against fp64
    over every grad, the bf16 copy against torch's cast everywhere, and sampled tensors -- the
    tied embedding (the largest) among them -- bit for bit against the oracle: master, m, v,
    bf16 copy and step counter."""
    import torchure_amd as ta

    shapes = shapes_for(config)
    g = torch.Generator(device=DEV).manual_seed(1)
    params = [torch.nn.Parameter(torch.randn(s, device=DEV, generator=g) * 0.02) for s in shapes]
    work = ta.attach_bf16_working_params(params)
    for w in work:
        w.grad = (torch.randn(w.shape, device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
    if config == "qwen3-0.6b":  # the 0.6B steady state has the clip not triggered: norm 0.5
        sq = sum(float(torch.sum(w.grad.double() ** 2).item()) for w in work)
        scale = 0.5 / math.sqrt(sq)
        for w in work:
            w.grad = (w.grad.float() * scale).to(torch.bfloat16)
    grads = [w.grad for w in work]
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})
    opt.init_state()  # the optimizer's pooled layout, filled in place with the steady state
    for p in params:
        st = opt.state[p]
        st["step"].fill_(1000.0)
        st["exp_avg"].copy_(torch.randn(p.shape, device=DEV, generator=g) * 1e-4)
        st["exp_avg_sq"].copy_(torch.randn(p.shape, device=DEV, generator=g).abs_() * 1e-8)
    for k in ("exp_avg", "exp_avg_sq"):  # one pool per role
        assert len({opt.state[p][k].untyped_storage().data_ptr() for p in params}) == 1
    sample = [0, 1, 5, 6, 200, len(shapes) - 1]

    def host(t):
        return t.detach().cpu().numpy().reshape(-1).copy()

    before = {i: (host(params[i]), host(opt.state[params[i]]["exp_avg"]),
                  host(opt.state[params[i]]["exp_avg_sq"]), H.from_dev_bf16(grads[i]).copy()) for i in sample}
    exact_sq = sum(float(torch.sum(gr.double() ** 2).item()) for gr in grads)
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    exact = math.sqrt(exact_sq)
    assert abs(norm.item() - exact) <= 1e-6 * exact
    if config == "qwen3-0.6b":
        assert abs(norm.item() - 0.5) < 1e-3 and coef.item() == 1.0
    else:
        assert 50.0 < norm.item() < 80.0 and coef.item() < 0.02
    for p, w in zip(params, work):
        assert torch.equal(w, p.detach().to(torch.bfloat16))
    for i in sample:
        p0, m0, v0, gb = before[i]
        out = np.zeros(p0.size, np.uint16)
        wd = 0.1 if len(shapes[i]) >= 2 else 0.0
        oracle.adamw_update_bf16(p0, m0, v0, gb, out, float(coef.item()), 1, 1001.0, 3e-4, 0.9, 0.95, wd,
                                 1e-8, threaded=True)
        st = opt.state[params[i]]
        assert np.array_equal(host(params[i]).view(np.int32), p0.view(np.int32)), i
        assert np.array_equal(host(st["exp_avg"]).view(np.int32), m0.view(np.int32)), i
        assert np.array_equal(host(st["exp_avg_sq"]).view(np.int32), v0.view(np.int32)), i
        assert np.array_equal(H.from_dev_bf16(work[i]), out), i
        assert st["step"].item() == 1001.0



@pytest.mark.parametrize("config", ["qwen3-0.6b", "qwen3-4b"])
def test_full_size_every_element_matches_torch_rocm_fused_adamw(config):
    """Every element of a full-size step (596M / 4.02B params, steady state, bf16 grads, clip 1.0
    triggered) against torch.optim.AdamW(fused=True) on the same GPU -- the reference's own
    optimizer -- fed the same inputs the reference trainer would give it: fp32 grads equal to the
    widened bf16 grads, scaled in place by the same clip coefficient (torch._foreach_mul_, the
    reference's clip). Masters, m, v and step counters bit for bit on every element, and the bf16
    working copies equal to torch's cast of torch's masters."""
    import torchure_amd as ta

    shapes = shapes_for(config)
    g = torch.Generator(device=DEV).manual_seed(5)
    params = [torch.nn.Parameter(torch.randn(s, device=DEV, generator=g) * 0.02) for s in shapes]
    work = ta.attach_bf16_working_params(params)
    for w in work:
        w.grad = (torch.randn(w.shape, device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})
    opt.init_state()  # the optimizer's pooled layout, filled in place with the steady state
    for p in params:
        st = opt.state[p]
        st["step"].fill_(1000.0)
        st["exp_avg"].copy_(torch.randn(p.shape, device=DEV, generator=g) * 1e-4)
        st["exp_avg_sq"].copy_(torch.randn(p.shape, device=DEV, generator=g).abs_() * 1e-8)
    for k in ("exp_avg", "exp_avg_sq"):  # one pool per role
        assert len({opt.state[p][k].untyped_storage().data_ptr() for p in params}) == 1
    ref = [torch.nn.Parameter(p.detach().clone()) for p in params]
    topt = torch.optim.AdamW([{"params": [q for q in ref if q.dim() >= 2], "weight_decay": 0.1},
                              {"params": [q for q in ref if q.dim() < 2], "weight_decay": 0.0}],
                             lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=True)
    for p, q, w in zip(params, ref, work):
        q.grad = w.grad.float()
        st, tst = opt.state[p], topt.state[q]
        tst["step"] = st["step"].clone()
        tst["exp_avg"] = st["exp_avg"].clone()
        tst["exp_avg_sq"] = st["exp_avg_sq"].clone()
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch._foreach_mul_([q.grad for q in ref], coef)
    topt.step()
    torch.cuda.synchronize()
    assert norm.item() > 1.0 and coef.item() < 1.0  # the clip triggered
    i32 = torch.int32
    for i, (p, q, w) in enumerate(zip(params, ref, work)):
        st, tst = opt.state[p], topt.state[q]
        assert torch.equal(p.detach().view(i32), q.detach().view(i32)), i
        assert torch.equal(st["exp_avg"].view(i32), tst["exp_avg"].view(i32)), i
        assert torch.equal(st["exp_avg_sq"].view(i32), tst["exp_avg_sq"].view(i32)), i
        assert st["step"].item() == tst["step"].item() == 1001.0
        assert torch.equal(w.detach().view(torch.int16), q.detach().to(torch.bfloat16).view(torch.int16)), i

def test_accumulate_list_fused_norm_and_reuse():
    """Micro-step accumulation: 4 bf16 micro-steps accumulated into fp32 .grad in one launch each;
    the last also yields the global norm, bit-identical to the standalone norm pass,
    and clip_grad_norm reuses it; the step then matches the oracle bit for bit."""
    import torchure_amd as ta
    from torchure_amd.core.grad_helper import grad_norm_launch
    from torchure_amd.optimizer.working import accumulate_grads_, cached_norm

    shapes = shapes_for("tiny") + [(1001,), (3, 333)]  # odd lengths exercise the tail
    host = H.make_host_set(shapes, seed=21)
    params, work, opt = H.device_setup(host, DEV)
    for w in work:
        w.grad = None
    r = H.rng(22)
    acc_ref = [np.zeros(numel(s), np.float32) for s in shapes]
    for k in range(4):
        for i, (s, w) in enumerate(zip(shapes, work)):
            if k == 3 and i == 5:
                continue  # no micro-grad for this param in the last step: still in the norm
            mg = oracle.bf16_rne((r.standard_normal(numel(s)) * 2e-3).astype(np.float32))
            acc_ref[i] = (acc_ref[i] + oracle.bf16_to_f32(mg)).astype(np.float32)
            w.grad = H.to_dev_bf16(mg, s, DEV)
        norm = accumulate_grads_(params, last=(k == 3))
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        assert np.array_equal(p.grad.cpu().numpy().reshape(-1), acc_ref[i]), i
        assert work[i].grad is None
    ref_norm, _ = grad_norm_launch([p.grad for p in params], None)
    assert norm.view(torch.int32).item() == ref_norm.view(torch.int32).item()
    exact = np.sqrt(sum(oracle.sumsq(a) for a in acc_ref))
    assert abs(norm.item() - exact) <= 1e-6 * exact
    assert cached_norm([p.grad for p in params]) is norm
    got = ta.clip_grad_norm(params, None, 1.0)
    assert got is norm
    coef = opt._pending[0].clone()
    assert float(coef.item()) == float(oracle.clip_coef(norm.item(), 1.0))
    opt.step()
    torch.cuda.synchronize()
    for i, h in enumerate(host):
        h["g"] = acc_ref[i]
    tens = H.oracle_tensors(host)
    oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
    w = H.compare_state(params, work, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w


def test_cached_norm_invalidated_by_inplace_change():
    import torchure_amd as ta
    from torchure_amd.optimizer.working import accumulate_grads_

    host = H.make_host_set([(64, 32), (100,)], seed=23)
    params, work, opt = H.device_setup(host, DEV)
    n1 = accumulate_grads_(params, last=True).item()
    params[0].grad.mul_(2.0)  # torch in-place op bumps the version: cache must not be used
    n2 = ta.clip_grad_norm(params, None, None).item()
    g0 = params[0].grad.double()
    g1 = params[1].grad.double()
    want = float(torch.sqrt((g0 * g0).sum() + (g1 * g1).sum()).item())
    assert abs(n2 - want) <= 1e-6 * want and abs(n2 - n1) > 1e-3 * n1


def test_accumulate_rejects_before_touching_any_grad():
    """A bad entry anywhere in the list raises before any p.grad is created or written,
    so the params ahead of it keep their grads (here: none, and one existing)."""
    from torchure_amd.optimizer.working import accumulate_grads_

    a = torch.nn.Parameter(torch.randn(64, device=DEV))
    b = torch.nn.Parameter(torch.randn(64, device=DEV))
    bad = torch.nn.Parameter(torch.randn(64, device=DEV, dtype=torch.float16))
    for p in (a, b, bad):
        w = torch.zeros(64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
        w.grad = torch.ones(64, device=DEV, dtype=torch.bfloat16)
        p._tm_working = w
    b.grad = torch.full((64,), 3.0, device=DEV)
    with pytest.raises(RuntimeError, match="float32"):
        accumulate_grads_([a, b, bad])
    assert a.grad is None
    assert torch.equal(b.grad, torch.full((64,), 3.0, device=DEV))
    assert a._tm_working.grad is not None and b._tm_working.grad is not None
    accumulate_grads_([a, b])
    assert torch.equal(a.grad, torch.ones(64, device=DEV))
    assert torch.equal(b.grad, torch.full((64,), 4.0, device=DEV))
    assert a._tm_working.grad is None and bad._tm_working.grad is not None


def test_ragged_full_size_three_chained_steps():
    """The ragged list at full size: 10,000 tensors, ~1.02e10 elements (~163 GB resident),
    ~30% odd lengths, 40% 1-D (no decay), 1% all-zero grads; three chained steps.
    Size-independent checks on every tensor (norm vs fp64, bf16 copy = torch's cast
    of the master, step counters) and bit-exact oracle checks on a sample that covers
    the largest, odd-length, 1-D and all-zero tensors, carried across the steps."""
    import torchure_amd as ta

    shapes = ragged_shapes()
    n_total = sum(numel(s) for s in shapes)
    assert len(shapes) == 10000 and n_total > 1e10
    gen = torch.Generator(device=DEV).manual_seed(5)
    params = [torch.nn.Parameter(torch.randn(s, device=DEV, generator=gen) * 0.02) for s in shapes]
    work = ta.attach_bf16_working_params(params)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})
    for p in params:
        st = opt.state[p]
        st["step"] = torch.tensor(1000.0, dtype=torch.float32, device=DEV)
        st["exp_avg"] = torch.randn(p.shape, device=DEV, generator=gen) * 1e-4
        st["exp_avg_sq"] = torch.randn(p.shape, device=DEV, generator=gen).abs_() * 1e-8
    zero = set(range(0, 10000, 100))
    sizes = [numel(s) for s in shapes]
    order = sorted(range(10000), key=lambda i: sizes[i])
    sample = sorted({order[-1], order[-2], order[0], 100, 200}
                    | {i for i in order[5000:5100] if sizes[i] % 8 and len(shapes[i]) == 1}
                    | {i for i in order[5000:5100] if sizes[i] % 4 == 1 and len(shapes[i]) == 2})
    held = {i: None for i in sample}
    for k in range(3):
        for i, w in enumerate(work):
            if w.grad is None:
                w.grad = torch.empty(w.shape, dtype=torch.bfloat16, device=DEV)
            if i in zero:
                w.grad.zero_()
            else:
                w.grad.normal_(0.0, 1e-3, generator=gen)
        for i in sample:
            st = opt.state[params[i]]
            held[i] = dict(p=params[i].detach().cpu().numpy().reshape(-1).copy(),
                           m=st["exp_avg"].cpu().numpy().reshape(-1).copy(),
                           v=st["exp_avg_sq"].cpu().numpy().reshape(-1).copy(),
                           g=H.from_dev_bf16(work[i].grad).copy())
        sq = torch.zeros((), dtype=torch.float64, device=DEV)
        for w in work:
            sq += torch.sum(w.grad.double() ** 2)
        norm = ta.clip_grad_norm(params, None, 1.0)
        coef = opt._pending[0].clone()
        opt.step()
        torch.cuda.synchronize()
        exact = float(sq.sqrt().item())
        print(f"ragged step {k}: norm {norm.item():.6f} (fp64 {exact:.6f}), coef {coef.item():.6f}", flush=True)
        assert abs(norm.item() - exact) <= 1e-6 * exact
        for p, w in zip(params, work):
            assert torch.equal(w, p.detach().to(torch.bfloat16))
        steps = torch.stack([opt.state[p]["step"] for p in params])
        assert bool(torch.all(steps == 1001.0 + k).item())
        for i in sample:
            h = held[i]
            wd = 0.1 if len(shapes[i]) >= 2 else 0.0
            out = np.zeros(h["p"].size, np.uint16)
            oracle.adamw_update_bf16(h["p"], h["m"], h["v"], h["g"], out, float(coef.item()), 1,
                                     1001.0 + k, 3e-4, 0.9, 0.95, wd, 1e-8)
            st = opt.state[params[i]]
            assert int(H.ulp_diff(params[i].detach().cpu().numpy().reshape(-1), h["p"]).max()) == 0, (k, i)
            assert np.array_equal(st["exp_avg"].cpu().numpy().reshape(-1), h["m"]), (k, i)
            assert np.array_equal(st["exp_avg_sq"].cpu().numpy().reshape(-1), h["v"]), (k, i)
            assert np.array_equal(H.from_dev_bf16(work[i]), out), (k, i)
    del params, work, opt
    torch.cuda.empty_cache()


def test_fresh_grads_each_step_two_optimizers_interleaved():
    """Grad tensors reallocated every step (set_to_none) on two interleaved optimizers,
    more steps than the uploader's pinned slots: every step matches the oracle, so no
    stale or foreign tensor table is ever used."""
    import torchure_amd as ta

    sets = []
    for seed in (31, 32):
        host = H.make_host_set([(96, 40), (257,), (1024, 3), (13,)], seed=seed)
        params, work, opt = H.device_setup(host, DEV)
        sets.append([host, params, work, opt, H.oracle_tensors(host)])
    r = H.rng(33)
    for k in range(6):
        for host, params, work, opt, tens in sets:
            opt.zero_grad()
            for i, h in enumerate(host):
                gb = oracle.bf16_rne((r.standard_normal(h["p"].size) * 1e-3).astype(np.float32))
                tens[i]["g"] = gb
                work[i].grad = H.to_dev_bf16(gb, h["shape"], DEV)
            ta.clip_grad_norm(params, None, 1.0)
            coef = opt._pending[0].clone()
            opt.step()
            torch.cuda.synchronize()
            oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
            w = H.compare_state(params, work, opt, tens)
            assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, (k, w)


def test_groups_with_different_hyperparameters():
    """Three param groups with different lr / weight decay / betas / eps in one launch."""
    import torchure_amd as ta

    host = H.make_host_set([(64, 16), (33,), (128, 8), (7, 7)], seed=34)
    params = [torch.nn.Parameter(torch.from_numpy(h["p"].copy()).view(h["shape"]).to(DEV)) for h in host]
    for p, h in zip(params, host):
        p.grad = torch.from_numpy(oracle.bf16_to_f32(h["g"]).copy()).view(h["shape"]).to(DEV)
    hp = [dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
          dict(lr=0.0, betas=(0.8, 0.9), eps=1e-6, weight_decay=0.5),
          dict(lr=5e-2, betas=(0.5, 0.75), eps=0.0, weight_decay=0.0)]
    groups = [dict(params=[params[0], params[1]], **hp[0]), dict(params=[params[2]], **hp[1]),
              dict(params=[params[3]], **hp[2])]
    opt = ta.AdamW(groups, fused=True)
    for p, h in zip(params, host):
        st = opt.state[p]
        st["step"] = torch.tensor(h["step"], dtype=torch.float32, device=DEV)
        st["exp_avg"] = torch.from_numpy(h["m"].copy()).view(h["shape"]).to(DEV)
        st["exp_avg_sq"] = torch.from_numpy(h["v"].copy()).view(h["shape"]).to(DEV)
    opt.step()
    torch.cuda.synchronize()
    gi_of = [0, 0, 1, 2]
    for i, (p, h) in enumerate(zip(params, host)):
        q = hp[gi_of[i]]
        t = dict(p=h["p"].copy(), m=h["m"].copy(), v=h["v"].copy())
        oracle.adamw_update(t["p"], t["m"], t["v"], oracle.bf16_to_f32(h["g"]).copy(), h["step"] + 1,
                            q["lr"], q["betas"][0], q["betas"][1], q["weight_decay"], q["eps"])
        st = opt.state[p]
        assert np.array_equal(p.detach().cpu().numpy().reshape(-1).view(np.int32), t["p"].view(np.int32)), i
        assert np.array_equal(st["exp_avg"].cpu().numpy().reshape(-1), t["m"]), i
        assert np.array_equal(st["exp_avg_sq"].cpu().numpy().reshape(-1), t["v"]), i


def test_nonfinite_grads_propagate_like_torch():
    """inf / NaN grads: same finiteness pattern and same finite values as torch-ROCm's
    fused AdamW on the same inputs (no clip, so the coefficient does not spread NaN)."""
    import torchure_amd as ta

    n = 4096
    r = H.rng(35)
    p0 = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    g[::97] = np.inf
    g[5::101] = -np.inf
    g[7::103] = np.nan
    mine = torch.nn.Parameter(torch.from_numpy(p0.copy()).to(DEV))
    ref = torch.nn.Parameter(torch.from_numpy(p0.copy()).to(DEV))
    mine.grad = torch.from_numpy(g.copy()).to(DEV)
    ref.grad = torch.from_numpy(g.copy()).to(DEV)
    o1 = ta.AdamW([mine], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=True)
    o2 = torch.optim.AdamW([ref], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=True)
    o1.step()
    o2.step()
    torch.cuda.synchronize()
    for a, b in ((mine.detach(), ref.detach()),
                 (o1.state[mine]["exp_avg"], o2.state[ref]["exp_avg"]),
                 (o1.state[mine]["exp_avg_sq"], o2.state[ref]["exp_avg_sq"])):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.array_equal(np.isnan(a), np.isnan(b))
        fin = np.isfinite(b)
        assert np.array_equal(np.isfinite(a), fin)
        assert np.array_equal(a[fin], b[fin])
        assert np.array_equal(a[np.isinf(b)], b[np.isinf(b)])


def test_checkpoint_file_roundtrip_continues_bit_exact(tmp_path):
    """torchure's Checkpointer flow (torch.save(optimizer.state_dict()); later
    torch.load(map_location="cpu", weights_only=True) + load_state_dict,
    torchure/checkpoint/checkpointer.py:43-60,81-82): a resumed optimizer continues
    exactly like the uninterrupted one."""
    import torchure_amd as ta

    host = H.make_host_set(shapes_for("tiny")[:6], seed=36)
    pa, wa, oa = H.device_setup(host, DEV)
    ta.clip_grad_norm(pa, None, 1.0)
    oa.step()
    torch.save(oa.state_dict(), tmp_path / "optimizer.pt")
    torch.save({"p": [p.detach().cpu() for p in pa]}, tmp_path / "model.pt")
    # uninterrupted second step
    ta.clip_grad_norm(pa, None, 1.0)
    oa.step()
    torch.cuda.synchronize()
    # resume from the files into fresh objects
    model = torch.load(tmp_path / "model.pt", map_location="cpu", weights_only=True)
    pb = [torch.nn.Parameter(t.to(DEV)) for t in model["p"]]
    wb = ta.attach_bf16_working_params(pb)
    for w, w0 in zip(wb, wa):
        w.grad = w0.grad.clone()
    ob = ta.build_optimizer(torch.nn.ParameterList(pb), "adamw",
                            {"lr": H.HYPER["lr"], "weight_decay": H.WD,
                             "betas": (H.HYPER["beta1"], H.HYPER["beta2"]), "fused": True})
    ob.load_state_dict(torch.load(tmp_path / "optimizer.pt", map_location="cpu", weights_only=True))
    ta.clip_grad_norm(pb, None, 1.0)
    ob.step()
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
        for k in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(oa.state[a][k], ob.state[b][k])
            assert ob.state[b][k].device == b.device


def test_pooled_state_checkpoint_size_and_torch_interop(tmp_path):
    """The lazy state is pooled (one fp32 buffer per role, each moment a view at the same
    distance from a 1 KiB boundary as its master, 16-byte aligned). torchure's Checkpointer flow still works both ways with torch.optim.AdamW
    (torchure/checkpoint/checkpointer.py:43-60,81-82): for the Qwen3-shaped set the saved file is
    not larger than the same state saved as separate tensors; torch's fused AdamW loads it with
    torch.load(weights_only=True) and continues bit for bit with this optimizer; and this
    optimizer loads torch's checkpoint back into its pooled layout and continues bit for bit."""
    import os

    import torchure_amd as ta

    shapes = shapes_for("tiny") + [(1001,), (3, 333), (128,), (7,)]
    gen = torch.Generator(device=DEV).manual_seed(43)
    init = [torch.randn(sh, device=DEV, generator=gen) * 0.02 for sh in shapes]
    grads = [[torch.randn(sh, device=DEV, generator=gen) * 1e-3 for sh in shapes] for _ in range(3)]

    def groups_of(ps):
        return [{"params": [p for p in ps if p.dim() >= 2], "weight_decay": 0.1},
                {"params": [p for p in ps if p.dim() < 2], "weight_decay": 0.0}]

    def ours(ps):
        return ta.build_optimizer(torch.nn.ParameterList(ps), "adamw",
                                  {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})

    def torch_fused(ps):
        return torch.optim.AdamW(groups_of(ps), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=True)

    def step(ps, opt, k):
        for p, g in zip(ps, grads[k]):
            p.grad = g.clone()
        opt.step()

    pa = [torch.nn.Parameter(t.clone()) for t in init]
    oa = ours(pa)
    step(pa, oa, 0)
    for k in ("exp_avg", "exp_avg_sq"):
        assert len({oa.state[p][k].untyped_storage().data_ptr() for p in pa}) == 1
    for p in pa:
        m, v = oa.state[p]["exp_avg"], oa.state[p]["exp_avg_sq"]
        assert m.data_ptr() % 1024 == v.data_ptr() % 1024
        assert m.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0
        if p.data_ptr() % 16 == 0 and p.numel() >= 256:  # the master's phase (from a 1 KiB boundary)
            assert m.data_ptr() % 1024 == p.data_ptr() % 1024

    # file size, on the Qwen3-shaped set alone (its moments need no padding in the pool)
    pq = [torch.nn.Parameter(torch.randn(sh, device=DEV, generator=gen) * 0.02) for sh in shapes_for("tiny")]
    oq = ours(pq)
    for p in pq:
        p.grad = torch.randn(p.shape, device=DEV, generator=gen) * 1e-3
    oq.step()
    sq = oq.state_dict()
    torch.save(sq, tmp_path / "pooled_q.pt")
    torch.save({"state": {i: {k: t.clone() for k, t in st.items()} for i, st in sq["state"].items()},
                "param_groups": sq["param_groups"]}, tmp_path / "separate_q.pt")
    assert os.path.getsize(tmp_path / "pooled_q.pt") <= os.path.getsize(tmp_path / "separate_q.pt")
    del pq, oq, sq

    sd = oa.state_dict()
    torch.save(sd, tmp_path / "pooled.pt")

    # torch's fused AdamW resumes from the pooled file and continues like this optimizer
    pb = [torch.nn.Parameter(p.detach().clone()) for p in pa]
    ob = torch_fused(pb)
    ob.load_state_dict(torch.load(tmp_path / "pooled.pt", map_location="cpu", weights_only=True))
    step(pa, oa, 1)
    step(pb, ob, 1)
    torch.cuda.synchronize()
    i32 = torch.int32
    for a, b in zip(pa, pb):
        assert torch.equal(a.detach().view(i32), b.detach().view(i32))
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(oa.state[a][k].view(i32), ob.state[b][k].view(i32))
        assert oa.state[a]["step"].item() == ob.state[b]["step"].item() == 2.0

    # and this optimizer resumes from torch's file, into its pooled layout
    torch.save(ob.state_dict(), tmp_path / "torch.pt")
    pc = [torch.nn.Parameter(p.detach().clone()) for p in pb]
    oc = ours(pc)
    oc.load_state_dict(torch.load(tmp_path / "torch.pt", map_location="cpu", weights_only=True))
    for k in ("exp_avg", "exp_avg_sq"):
        assert len({oc.state[p][k].untyped_storage().data_ptr() for p in pc}) == 1
    step(pb, ob, 2)
    step(pc, oc, 2)
    torch.cuda.synchronize()
    for b, c in zip(pb, pc):
        assert torch.equal(b.detach().view(i32), c.detach().view(i32))
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(ob.state[b][k].view(i32), oc.state[c][k].view(i32))
        assert oc.state[c]["step"].item() == 3.0 and oc.state[c]["step"].device == c.device


def test_checkpoint_from_non_fused_torch_adamw(tmp_path):
    """A checkpoint written by torch's default (foreach, non-fused) AdamW keeps `step` as a
    CPU tensor and `fused=None` in its groups, so torch's load policy leaves `step` where it
    is (torch/optim/optimizer.py:770-799) and copies `fused=None` over the loading
    optimizer's groups (torch's own fused AdamW then continues with the foreach recipe).
    Loaded into this AdamW, the groups say fused again, the first step moves `step` to the
    param's device as fp32, and the result equals torch's fused AdamW given the same state
    (its groups set back to fused and its steps moved to the device, which its fused path
    needs)."""
    import torchure_amd as ta

    gen = torch.Generator(device=DEV).manual_seed(41)
    shapes = [(64, 32), (32,), (17, 5)]
    init = [torch.randn(s, device=DEV, generator=gen) * 0.02 for s in shapes]
    grads = [[torch.randn(s, device=DEV, generator=gen) * 1e-3 for s in shapes] for _ in range(3)]

    def groups_of(ps):
        return [{"params": [p for p in ps if p.dim() >= 2], "weight_decay": 0.1},
                {"params": [p for p in ps if p.dim() < 2], "weight_decay": 0.0}]

    src = [torch.nn.Parameter(t.clone()) for t in init]
    topt = torch.optim.AdamW(groups_of(src), lr=3e-4, betas=(0.9, 0.95))  # foreach on the GPU
    for k in range(2):
        for p, g in zip(src, grads[k]):
            p.grad = g.clone()
        topt.step()
    sd = topt.state_dict()
    assert all(st["step"].device.type == "cpu" for st in sd["state"].values())
    torch.save(sd, tmp_path / "optimizer.pt")

    def resumed(make):
        ps = [torch.nn.Parameter(p.detach().clone()) for p in src]
        opt = make(ps)
        opt.load_state_dict(torch.load(tmp_path / "optimizer.pt", map_location="cpu", weights_only=True))
        for p, g in zip(ps, grads[2]):
            p.grad = g.clone()
        opt.step()
        return ps, opt

    mine, mopt = resumed(lambda ps: ta.build_optimizer(torch.nn.ParameterList(ps), "adamw",
                                                       {"lr": 3e-4, "weight_decay": 0.1,
                                                        "betas": (0.9, 0.95), "fused": True}))
    def fused_torch(ps):
        opt = torch.optim.AdamW(groups_of(ps), lr=3e-4, betas=(0.9, 0.95), fused=True)
        load = opt.load_state_dict

        def load_as_fused(sd):
            load(sd)
            for g in opt.param_groups:
                g["fused"], g["foreach"] = True, None
            for st in opt.state.values():
                st["step"] = st["step"].to(device=DEV, dtype=torch.float32)
        opt.load_state_dict = load_as_fused
        return opt

    ref, ropt = resumed(fused_torch)
    assert all(g["fused"] is True and g["foreach"] is None for g in mopt.state_dict()["param_groups"])
    torch.cuda.synchronize()
    for a, b in zip(mine, ref):
        assert torch.equal(a, b)
        sa, sb = mopt.state[a], ropt.state[b]
        assert sa["step"].device == a.device and sa["step"].dtype == torch.float32
        assert sa["step"].item() == 3.0 and sb["step"].item() == 3.0
        assert torch.equal(sa["exp_avg"], sb["exp_avg"]) and torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"])


def test_grads_as_views_into_flat_buckets():
    """DDP-style flat grad buckets (torchure/parallelism/data_parallel.py:53-66): grads
    are views into one flat fp32 buffer at arbitrary offsets, including ones that
    break 16-byte alignment; the tables alias them directly."""
    import torchure_amd as ta

    shapes = [(64, 32), (17,), (100, 3), (5,), (8, 8)]
    host = H.make_host_set(shapes, seed=37, grad_dtype="f32")
    params = [torch.nn.Parameter(torch.from_numpy(h["p"].copy()).view(h["shape"]).to(DEV)) for h in host]
    total = sum(h["p"].size for h in host)
    bucket = torch.zeros(total + 3, device=DEV)
    off = 0
    for p, h in zip(params, host):
        view = bucket[off:off + h["p"].size].view(h["shape"])
        view.copy_(torch.from_numpy(h["g"]).view(h["shape"]))
        p.grad = view
        off += h["p"].size
    opt = ta.AdamW(params, lr=H.HYPER["lr"], betas=(H.HYPER["beta1"], H.HYPER["beta2"]),
                   weight_decay=H.WD, fused=True)
    for p, h in zip(params, host):
        st = opt.state[p]
        st["step"] = torch.tensor(h["step"], dtype=torch.float32, device=DEV)
        st["exp_avg"] = torch.from_numpy(h["m"].copy()).view(h["shape"]).to(DEV)
        st["exp_avg_sq"] = torch.from_numpy(h["v"].copy()).view(h["shape"]).to(DEV)
        h["wd"] = H.WD
    norm = ta.clip_grad_norm(params, None, 1.0)
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    tens = H.oracle_tensors(host)
    for t in tens:
        t["out"] = None
    ref_norm, _ = oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
    assert abs(norm.item() - float(ref_norm)) <= 1e-6 * float(ref_norm)
    w = H.compare_state(params, None, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w


def test_two_optimizers_on_two_streams_concurrently():
    """Two independent optimizers whose clip + step calls are issued interleaved on two
    streams (default priority) give the same bits as running them one after the other on
    the default stream: the tables, workspaces and staging buffers of one call are never
    reused by the other's while it may still read them."""
    import torchure_amd as ta

    def setups():
        a = H.device_setup(H.make_host_set(shapes_for("tiny"), seed=61), DEV)
        b = H.device_setup(H.make_host_set(shapes_for("tiny")[::-1], seed=62), DEV)
        return a, b

    def run(pairs, streams):
        for _ in range(3):
            for (params, work, opt), s in zip(pairs, streams):
                with torch.cuda.stream(s):
                    ta.clip_grad_norm(params, None, 1.0)
                    opt.step()
        torch.cuda.synchronize()

    seq = setups()
    run(seq, [torch.cuda.current_stream(), torch.cuda.current_stream()])
    con = setups()
    torch.cuda.synchronize()
    run(con, [torch.cuda.Stream(), torch.cuda.Stream()])
    for (pa, wa, oa), (pb, wb, ob) in zip(seq, con):
        for x, y, u, v in zip(pa, pb, wa, wb):
            assert torch.equal(x, y)
            assert torch.equal(u.view(torch.int16), v.view(torch.int16))
            for k in ("step", "exp_avg", "exp_avg_sq"):
                assert torch.equal(oa.state[x][k], ob.state[y][k])


def test_shared_params_clip_in_place():
    """Params held by two optimizers: the clip scales their grads in place (no deferral into
    one optimizer), so both steps read the clipped grads, as with the reference's in-place
    clip. Checked bit for bit against the same sequence with defer_clip=False."""
    import torchure_amd as ta

    def run(defer):
        gen = torch.Generator(device=DEV).manual_seed(8)
        shared = torch.nn.Parameter(torch.randn(64, 32, device=DEV, generator=gen) * 0.02)
        own = torch.nn.Parameter(torch.randn(100, device=DEV, generator=gen) * 0.02)
        shared.grad = torch.randn(64, 32, device=DEV, generator=gen)
        own.grad = torch.randn(100, device=DEV, generator=gen)
        o1 = ta.AdamW([shared, own], lr=1e-3, defer_clip=defer)
        o2 = ta.AdamW([shared], lr=2e-3, defer_clip=defer)
        norm = ta.clip_grad_norm([shared, own], None, 1.0)
        assert o1._pending is None and o2._pending is None
        o1.step()
        o2.step()
        torch.cuda.synchronize()
        return norm, shared.detach().clone(), own.detach().clone(), shared.grad.clone()

    a, b = run(True), run(False)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert a[0].item() > 1.0  # the clip was active


def test_sparse_grads_are_refused():
    """A sparse grad (nn.Embedding(sparse=True)) is refused with torch's AdamW message by the
    step, and with a clear message by the clip, before any kernel runs."""
    import torchure_amd as ta

    emb = torch.nn.Embedding(50, 8, sparse=True).to(DEV)
    emb(torch.tensor([1, 2, 3], device=DEV)).sum().backward()
    assert emb.weight.grad.is_sparse
    opt = ta.AdamW(emb.parameters())
    with pytest.raises(RuntimeError, match="does not support sparse gradients"):
        opt.step()
    with pytest.raises(RuntimeError, match="dense grads only"):
        ta.clip_grad_norm(emb.parameters(), None, 1.0)


def test_eager_scale_matches_foreach_mul():
    """The eager clip's in-place scale against torch._foreach_mul_ with the same 0-d device
    coefficient (torchure/core/grad_helper.py:33), bit for bit, for fp32 and bf16 grads:
    lengths of 1, 7, 1000, one chunk + 5 and 40,000 elements, lengths around the kernel's
    512-element slice and its two 256-element halves (255, 257, 300, 511, 513, 770), and views
    at offsets that are not 16-byte aligned, so the vector, tail and element-wise paths all
    run."""
    from torchure_amd.core.grad_helper import scale_grads_

    gen = torch.Generator(device=DEV).manual_seed(77)
    for dtype in (torch.float32, torch.bfloat16):
        base = (torch.randn(200_000, device=DEV, generator=gen) * 3.0).to(dtype)
        base[5] = float("inf")
        base[6] = float("nan")
        base[7] = -0.0
        grads = [base[0:1], base[16:23], base[32:1032], base[2048:2048 + 16384 + 5],
                 base[50_000:90_000], base[100_001:100_001 + 5000], base[110_003:110_003 + 33]]
        grads += [base[o:o + n] for o, n in ((120_000, 255), (121_000, 257), (122_000, 300),
                                             (123_000, 511), (124_000, 513), (125_008, 770))]
        ref = [g.clone() for g in grads]
        coef = torch.tensor(0.3712, device=DEV)
        scale_grads_(grads, coef)
        torch._foreach_mul_(ref, coef)
        for g, r in zip(grads, ref):
            bits = torch.int32 if dtype == torch.float32 else torch.int16
            assert torch.equal(g.view(bits), r.view(bits)), (dtype, g.numel())


def test_materialize_clip_equals_eager_clip():
    import torchure_amd as ta

    host = H.make_host_set([(64, 64), (50,)], seed=38, grad_std=0.1, grad_dtype="f32")
    pa, _, oa = H.device_setup(host, DEV, working=False)
    pb, _, ob = H.device_setup(host, DEV, working=False)
    ob.defer_clip = False
    ta.clip_grad_norm(pa, None, 1.0)
    assert oa._pending is not None
    oa.materialize_clip()
    ta.clip_grad_norm(pb, None, 1.0)
    assert ob._pending is None
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a.grad, b.grad)


def test_deferred_clip_leaves_grads_unscaled_until_step():
    """The documented drop-in difference of the deferred clip (the default): between
    clip_grad_norm and step(), p.grad still reads the unscaled values, where the reference's
    clip has already scaled them in place (torchure/core/grad_helper.py:32-33). The step
    applies the scale; materialize_clip() applies it to p.grad on request, giving the
    in-place clip's values; with defer_clip=False the clip scales p.grad at once."""
    import torchure_amd as ta

    host = H.make_host_set([(64, 64), (50,)], seed=39, grad_std=0.1, grad_dtype="f32")
    pd, _, od = H.device_setup(host, DEV, working=False)
    pe, _, oe = H.device_setup(host, DEV, working=False)
    oe.defer_clip = False
    raw = [p.grad.clone() for p in pd]
    ta.clip_grad_norm(pd, None, 1.0)
    ta.clip_grad_norm(pe, None, 1.0)
    torch.cuda.synchronize()
    coef = od._pending[0].item()
    assert coef < 1.0
    for p, g in zip(pd, raw):  # deferred: unscaled until the step
        assert torch.equal(p.grad, g)
    for p, g in zip(pe, raw):  # eager (the reference's behaviour): scaled in place
        assert torch.equal(p.grad, g * torch.tensor(coef, device=DEV))
    od.materialize_clip()
    torch.cuda.synchronize()
    for a, b in zip(pd, pe):
        assert torch.equal(a.grad, b.grad)


@pytest.mark.parametrize("route", ["eager", "materialize"])
def test_bf16_grads_deferred_and_in_place_clip(route):
    """bf16 working-copy grads take one of two clip routes, each checked against its own
    definition. The deferred clip multiplies float(g) by the fp32 coefficient inside the
    update. That is the oracle's step on bf16 grads and the reference trainer's arithmetic:
    autocast makes its fp32 grads float(bf16 grad), and _foreach_mul_ scales them in fp32
    (grad_helper.py:33). An in-place scale of bf16 grads (defer_clip=False, or
    materialize_clip()) has to store bf16. It is torch._foreach_mul_ on the bf16 list, which
    rounds the coefficient and the product to bf16, and the step then reads those grads
    unscaled. Both routes give the same norm; their params differ by that rounding."""
    import torchure_amd as ta

    host = H.make_host_set([(256, 192), (1000,), (77,)], seed=41, grad_std=0.05)
    pa, wa, oa = H.device_setup(host, DEV)
    norm_a = ta.clip_grad_norm(pa, None, 1.0)
    coef = oa._pending[0].clone()
    assert float(coef.item()) < 1.0  # the clip is active
    oa.step()
    tens = H.oracle_tensors(host)
    oracle.reference_step(tens, H.HYPER, 1.0, clip_override=float(coef.item()))
    w = H.compare_state(pa, wa, oa, tens)
    assert w["p"] <= 2 and w["m"] <= 2 and w["v"] <= 2 and w["bf16"] == 0, w

    pb, wb, ob = H.device_setup(host, DEV)
    if route == "eager":
        ob.defer_clip = False
    grads0 = [x.grad.clone() for x in wb]
    norm_b = ta.clip_grad_norm(pb, None, 1.0)
    if route == "materialize":
        assert ob._pending is not None
        ob.materialize_clip()
    assert ob._pending is None
    assert norm_b.view(torch.int32).item() == norm_a.view(torch.int32).item()
    ref = [g.clone() for g in grads0]
    torch._foreach_mul_(ref, coef)
    for x, r in zip(wb, ref):
        assert torch.equal(x.grad.view(torch.int16), r.view(torch.int16))
    ob.step()
    tens_b = H.oracle_tensors(host)
    for t, r in zip(tens_b, ref):
        t["g"] = H.from_dev_bf16(r)
    oracle.reference_step(tens_b, H.HYPER, None)
    w = H.compare_state(pb, wb, ob, tens_b)
    assert w["p"] <= 2 and w["m"] <= 2 and w["v"] <= 2 and w["bf16"] == 0, w
    torch.cuda.synchronize()
    assert any(not torch.equal(a, b) for a, b in zip(pa, pb))


def test_step_bumps_autograd_versions():
    """The kernels write through raw pointers; the step bumps the version counters of
    everything it wrote, as torch's in-place fused AdamW does, so autograd still
    detects a param modified between forward and backward."""
    import torchure_amd as ta

    host = H.make_host_set([(32, 16), (9,)], seed=39)
    params, work, opt = H.device_setup(host, DEV)
    before = [(p._version, w._version, opt.state[p]["exp_avg"]._version) for p, w in zip(params, work)]
    x = torch.randn(4, 32, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = (x @ work[0]).sum()  # saves work[0] (for x's grad) for backward
    opt.step()
    for (pv, wv, mv), p, w in zip(before, params, work):
        assert p._version > pv and w._version > wv and opt.state[p]["exp_avg"]._version > mv
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        y.backward()


def test_state_storage_swapped_between_steps():
    """`.data =` on a state tensor or a working copy replaces its storage (the old one is
    freed) without changing the object; the next step must write the new storage.
    Checked against an identical optimizer whose tensors were left alone."""
    host = H.make_host_set([(64, 48), (33,), (8, 8)], seed=41)
    a_params, a_work, a_opt = H.device_setup(host, DEV)
    b_params, b_work, b_opt = H.device_setup(host, DEV)
    a_opt.step()
    b_opt.step()
    # the master keeps its storage, so only the new checks can notice each swap
    st0, st2 = a_opt.state[a_params[0]], a_opt.state[a_params[2]]
    for k in ("exp_avg", "exp_avg_sq", "step"):
        st0[k].data = st0[k].data.clone()
    a_work[1].data = a_work[1].data.clone()
    st2["exp_avg_sq"].data = st2["exp_avg_sq"].data.clone()
    torch.cuda.synchronize()
    a_opt.step()
    b_opt.step()
    torch.cuda.synchronize()
    for (p, w), (q, u) in zip(zip(a_params, a_work), zip(b_params, b_work)):
        assert torch.equal(p, q) and torch.equal(w, u)
        for k in ("exp_avg", "exp_avg_sq", "step"):
            assert torch.equal(a_opt.state[p][k], b_opt.state[q][k]), k


def _clip_setup(defer):
    import torchure_amd as ta

    host = H.make_host_set([(64, 48), (33,), (8, 8)], seed=43)
    params, work, opt = H.device_setup(host, DEV, grad_on_master=True)
    opt.defer_clip = defer
    norm = ta.clip_grad_norm(params, None, 0.01)  # clips
    return params, opt, norm


def test_deferred_clip_rejects_grads_modified_in_place():
    """The reference scales at clip time; a grad changed in place before the step cannot
    be reproduced by scaling later, so the deferred path raises instead of diverging."""
    params, opt, _ = _clip_setup(True)
    before = [p.detach().clone() for p in params]
    params[1].grad.add_(1.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        opt.step()
    # the clip stays pending: a second step is refused too, not run on unscaled grads
    with pytest.raises(RuntimeError, match="modified in place"):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(p, b) for p, b in zip(params, before))
    opt.zero_grad()  # drops the pending clip with the grads
    assert opt._pending is None
    params, opt, _ = _clip_setup(True)
    params[0].grad.mul_(2.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        opt.materialize_clip()
    with pytest.raises(RuntimeError, match="modified in place"):
        opt.step()


def test_deferred_clip_with_replaced_grad_matches_eager():
    """A grad replaced by a new tensor after the clip steps unscaled (the reference
    scaled the old tensor); the others step clipped. Bit-exact against the eager path."""
    runs = []
    for defer in (True, False):
        params, opt, norm = _clip_setup(defer)
        g = torch.Generator(device=DEV).manual_seed(5)
        params[2].grad = torch.randn(params[2].shape, device=DEV, generator=g)
        opt.step()
        torch.cuda.synchronize()
        runs.append(([p.detach().clone() for p in params],
                     [opt.state[p]["exp_avg"].clone() for p in params], norm.clone()))
    (pa, ma, na), (pb, mb, nb) = runs
    assert torch.equal(na, nb)
    for x, y in zip(pa + ma, pb + mb):
        assert torch.equal(x, y)


def test_accumulated_grads_equal_autograd_under_autocast():
    """Micro-step accumulation against torch's own autograd, bit for bit. Reference:
    fp32 params under bf16 autocast (torchure/train/trainer.py:372-390): autocast casts
    each weight to bf16 (RNE), the cast's backward widens the bf16 grad, the first
    backward assigns p.grad and later ones add to it. This build: bf16 working copies
    (RNE of the masters), bf16 grads on them, accumulate_grads_ after each backward.
    Then the assignment itself on special values: a first micro-grad of -0 stays -0
    (0 + -0 would give +0), NaN and infinities widen unchanged."""
    import torchure_amd as ta
    from torchure_amd.optimizer.working import accumulate_grads_

    torch.manual_seed(3)
    shapes = [(96, 64), (64, 96), (40, 64)]
    ref = [torch.nn.Parameter(torch.randn(s, device=DEV) * 0.05) for s in shapes]
    mine = [torch.nn.Parameter(p.detach().clone()) for p in ref]
    work = ta.attach_bf16_working_params(mine)
    micro = 3
    g = torch.Generator(device=DEV).manual_seed(8)
    xs = [torch.randn(32, 64, device=DEV, generator=g) for _ in range(micro)]

    def forward(ws, x):
        h = torch.nn.functional.silu(torch.nn.functional.linear(x, ws[0]))
        h = torch.nn.functional.linear(h, ws[1])
        return torch.nn.functional.linear(h, ws[2]).float().square().mean() / micro

    for x in xs:
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            forward(ref, x).backward()
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            forward(work, x.to(torch.bfloat16)).backward()
        accumulate_grads_(mine)
    torch.cuda.synchronize()
    for a, b in zip(mine, ref):
        assert torch.equal(a.grad.view(torch.int32), b.grad.view(torch.int32))

    bits = np.array([0x8000, 0x0000, 0x7FC0, 0x7F80, 0xFF80, 0x3FC0, 0x0001] * 5, dtype=np.uint16)
    q = torch.nn.Parameter(torch.zeros(bits.size, device=DEV))
    (w,) = ta.attach_bf16_working_params([q])
    w.grad = torch.from_numpy(bits.view(np.int16).copy()).to(DEV).view(torch.bfloat16)
    accumulate_grads_([q])
    got = q.grad.view(torch.int32).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_stale_working_copy_detected_and_refreshed():
    """Masters changed outside the step (a resume via model.load_state_dict) leave the
    bf16 working copies stale: the step raises instead of training on a forward that used
    old weights; refresh_bf16_working_params rewrites them as RNE(master) and the step
    then matches an optimizer built fresh on the new masters."""
    import torchure_amd as ta

    host = H.make_host_set([(64, 48), (33,)], seed=44)
    params, work, opt = H.device_setup(host, DEV)
    opt.step()
    new = [torch.randn(p.shape, device=DEV) * 0.02 for p in params]
    model = torch.nn.ParameterList(params)
    model.load_state_dict({str(i): t for i, t in enumerate(new)})
    grads = [w.grad.clone() for w in work]
    with pytest.raises(RuntimeError, match="stale"):
        opt.step()
    ta.refresh_bf16_working_params(params)
    for p, w in zip(params, work):
        assert torch.equal(w, p.detach().to(torch.bfloat16))
    ref_params, ref_work, ref_opt = H.device_setup(host, DEV)
    # deep copy: load_state_dict keeps device tensors as they are, which would alias the state
    ref_opt.load_state_dict(copy.deepcopy(opt.state_dict()))
    for p, q, w, g in zip(ref_params, new, ref_work, grads):
        with torch.no_grad():
            p.copy_(q)
        w.grad = g
    ta.refresh_bf16_working_params(ref_params)
    opt.step()
    ref_opt.step()
    torch.cuda.synchronize()
    for p, q, w, u in zip(params, ref_params, work, ref_work):
        assert torch.equal(p, q) and torch.equal(w, u)


def test_cached_plan_follows_group_list_edits():
    """Steady-state steps reuse the previous step's table; a param replaced inside a group's
    list (same length) must be the one updated next, and the old one left alone."""
    host = H.make_host_set([(32, 16), (16,)], seed=45)
    params, work, opt = H.device_setup(host, DEV, grad_on_master=True)
    opt.step()
    opt.step()  # second step: served from the cached plan
    old = params[0]
    new = torch.nn.Parameter(torch.randn_like(old))
    new.grad = torch.randn_like(old) * 1e-3
    opt.param_groups[0]["params"][0] = new
    before_old, before_new = old.detach().clone(), new.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert torch.equal(old, before_old)
    assert not torch.equal(new, before_new)
    assert float(opt.state[new]["step"]) == 1.0


def test_steady_state_transitions_match_torch():
    """Steps served from the cached plan and steps that must leave it, against torch's
    fused AdamW, bit for bit: grads reused in place (zero_grad(set_to_none=False)), a param
    whose grad disappears for a step (a frozen layer), fresh grad tensors, and the clip."""
    import torchure_amd as ta

    torch.manual_seed(12)
    shapes = [(48, 32), (32,), (16, 8), (8,)]
    init = [torch.randn(sh, device=DEV) * 0.05 for sh in shapes]
    mine = [torch.nn.Parameter(t.clone()) for t in init]
    ref = [torch.nn.Parameter(t.clone()) for t in init]
    groups = lambda ps: [{"params": [p for p in ps if p.dim() >= 2], "weight_decay": 0.1},
                         {"params": [p for p in ps if p.dim() < 2], "weight_decay": 0.0}]
    opt = ta.AdamW(groups(mine), lr=1e-3, betas=(0.9, 0.95), fused=True)
    opt_r = torch.optim.AdamW(groups(ref), lr=1e-3, betas=(0.9, 0.95), fused=True)
    g = torch.Generator(device=DEV).manual_seed(3)
    for k in range(7):
        grads = [torch.randn(sh, device=DEV, generator=g) * 1e-3 for sh in shapes]
        for i, (a, b) in enumerate(zip(mine, ref)):
            frozen = k == 3 and i == 2
            if frozen:
                a.grad = b.grad = None
            elif k < 4 and a.grad is not None:  # in place, as after zero_grad(set_to_none=False)
                a.grad.copy_(grads[i])
                b.grad.copy_(grads[i])
            else:
                a.grad, b.grad = grads[i].clone(), grads[i].clone()
        ta.clip_grad_norm(mine, None, 1e9)  # coefficient 1.0, deferred into the step
        torch.nn.utils.clip_grad_norm_(ref, 1e9)
        opt.step()
        opt_r.step()
    torch.cuda.synchronize()
    for a, b in zip(mine, ref):
        assert torch.equal(a, b)
        for key in ("exp_avg", "exp_avg_sq", "step"):
            assert torch.equal(opt.state[a][key], opt_r.state[b][key]), key


def test_tensor_beyond_2_31_elements():
    """One tensor of 2^31 + 12,345 elements (odd: the element-wise tail runs too), the
    64-bit addressing of every kernel on the path: attach (cast), clip (norm + deferred
    coefficient) and the step. Windows at the start, across element 2^31 and at the end are
    checked bit for bit against the oracle; the norm against fp64 over every element."""
    import torchure_amd as ta

    n = 2**31 + 12345
    g = torch.Generator(device=DEV).manual_seed(31)
    p = torch.nn.Parameter(torch.randn((1, n), device=DEV, generator=g) * 0.02)
    (w,) = ta.attach_bf16_working_params([p])
    w.grad = (torch.randn((1, n), device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
    opt = ta.AdamW([p], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=True)
    st = opt.state[p]
    st["step"] = torch.tensor(1000.0, device=DEV)
    st["exp_avg"] = torch.randn((1, n), device=DEV, generator=g) * 1e-4
    st["exp_avg_sq"] = torch.randn((1, n), device=DEV, generator=g).abs_() * 1e-8
    wins = [(0, 40000), (2**31 - 20000, 2**31 + 10000), (n - 40001, n)]
    assert all(0 <= a < b <= n for a, b in wins)
    flat = lambda t: t.detach().reshape(-1)
    before = [(flat(p)[a:b].cpu().numpy().copy(), flat(st["exp_avg"])[a:b].cpu().numpy().copy(),
               flat(st["exp_avg_sq"])[a:b].cpu().numpy().copy(),
               flat(w.grad)[a:b].view(torch.int16).cpu().numpy().view(np.uint16).copy()) for a, b in wins]
    norm = ta.clip_grad_norm([p], None, 1.0)
    coef = float(opt._pending[0].item())
    opt.step()
    torch.cuda.synchronize()
    gr = flat(w.grad)
    exact = sum(float((gr[s:s + 2**28].double() ** 2).sum()) for s in range(0, n, 2**28))
    assert abs(norm.item() - np.sqrt(exact)) <= 1e-6 * np.sqrt(exact)
    assert coef < 1.0
    for (a, b), (p0, m0, v0, g0) in zip(wins, before):
        assert p0.size == b - a
        out = np.zeros(b - a, np.uint16)
        oracle.adamw_update_bf16(p0, m0, v0, g0, out, coef, True, 1001.0, 3e-4, 0.9, 0.95, 0.1, 1e-8)
        assert np.array_equal(flat(p)[a:b].cpu().numpy(), p0), (a, b)
        assert np.array_equal(flat(st["exp_avg"])[a:b].cpu().numpy(), m0), (a, b)
        assert np.array_equal(flat(st["exp_avg_sq"])[a:b].cpu().numpy(), v0), (a, b)
        assert np.array_equal(flat(w)[a:b].view(torch.int16).cpu().numpy().view(np.uint16), out), (a, b)
    assert float(st["step"]) == 1001.0
    del p, w, opt, st, gr
    torch.cuda.empty_cache()


def test_full_size_config3_fp32_accumulation():
    """Grad accumulation at full size (Qwen3-0.6B shapes, 596M params): four bf16 micro-steps
    accumulated into fp32 .grad (the last one also measuring the norm), grads scaled
    so the global norm is ~5 and the clip triggers, WSD lr at decay step 9800. The
    fused norm equals the standalone norm pass bit for bit and fp64 within 1e-6;
    sampled tensors match the oracle bit for bit."""
    import torchure_amd as ta
    from torchure_amd.core.grad_helper import grad_norm_launch
    from torchure_amd.optimizer.working import accumulate_grads_

    shapes = shapes_for("qwen3-0.6b")
    gen = torch.Generator(device=DEV).manual_seed(3)
    params = [torch.nn.Parameter(torch.randn(s, device=DEV, generator=gen) * 0.02) for s in shapes]
    work = ta.attach_bf16_working_params(params)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True})
    sched = ta.build_scheduler(opt, {"type": "wsd", "total_steps": 10000, "warmup_ratio": 0.001,
                                     "decay_ratio": 0.2})
    sched.last_epoch = 9799
    sched.step()
    lr = opt.param_groups[0]["lr"]
    assert lr == 3e-4 * oracle.wsd_scale(9800, 10000, 0.001, 0.2)
    for p in params:
        st = opt.state[p]
        st["step"] = torch.tensor(9799.0, dtype=torch.float32, device=DEV)
        st["exp_avg"] = torch.randn(p.shape, device=DEV, generator=gen) * 1e-4
        st["exp_avg_sq"] = torch.randn(p.shape, device=DEV, generator=gen).abs_() * 1e-8
    # sigma so that 4 summed micro-grads have global norm ~5: 5 / sqrt(4 * N)
    sigma = 5.0 / np.sqrt(4.0 * sum(numel(s) for s in shapes))
    sample = [0, 3, 5, 6, len(shapes) - 1]
    micro_host = {i: [] for i in sample}
    for k in range(4):
        for i, w in enumerate(work):
            w.grad = (torch.randn(w.shape, device=DEV, generator=gen) * sigma).to(torch.bfloat16)
            if i in micro_host:
                micro_host[i].append(H.from_dev_bf16(w.grad).copy())
        if k == 3:
            before = {i: (params[i].detach().cpu().numpy().reshape(-1).copy(),
                          opt.state[params[i]]["exp_avg"].cpu().numpy().reshape(-1).copy(),
                          opt.state[params[i]]["exp_avg_sq"].cpu().numpy().reshape(-1).copy())
                      for i in sample}
        norm = accumulate_grads_(params, last=(k == 3))
    grads = [p.grad for p in params]
    standalone, _ = grad_norm_launch(grads, None)
    exact_sq = sum(float(torch.sum(g.double() ** 2).item()) for g in grads)
    torch.cuda.synchronize()
    assert norm.view(torch.int32).item() == standalone.view(torch.int32).item()
    assert abs(norm.item() - np.sqrt(exact_sq)) <= 1e-6 * np.sqrt(exact_sq)
    assert 4.0 < norm.item() < 6.0
    acc = {i: params[i].grad.cpu().numpy().reshape(-1).copy() for i in sample}
    got = ta.clip_grad_norm(params, None, 1.0)
    assert got is norm
    coef = opt._pending[0].clone()
    opt.step()
    torch.cuda.synchronize()
    assert float(coef.item()) < 0.25
    for i in sample:
        want = np.zeros_like(acc[i])
        for mg in micro_host[i]:
            want = (want + oracle.bf16_to_f32(mg)).astype(np.float32)
        assert np.array_equal(acc[i], want), i
        p0, m0, v0 = before[i]
        gclip = (acc[i] * np.float32(coef.item())).astype(np.float32)
        wd = 0.1 if len(shapes[i]) >= 2 else 0.0
        oracle.adamw_update(p0, m0, v0, gclip, 9800.0, lr, 0.9, 0.95, wd, 1e-8, threaded=True)
        st = opt.state[params[i]]
        assert int(H.ulp_diff(params[i].detach().cpu().numpy().reshape(-1), p0).max()) == 0, i
        assert np.array_equal(st["exp_avg"].cpu().numpy().reshape(-1), m0), i
        assert np.array_equal(st["exp_avg_sq"].cpu().numpy().reshape(-1), v0), i
        assert torch.equal(work[i], params[i].detach().to(torch.bfloat16))
    del params, work, opt, grads
    torch.cuda.empty_cache()


class _TiedLM(torch.nn.Module):
    """A small language model with a tied embedding / output head: the parameter
    reached through two modules must count once (model.parameters() yields it once)."""

    def __init__(self, vocab=64, dim=32):
        super().__init__()
        self.emb = torch.nn.Embedding(vocab, dim)
        self.norm1 = torch.nn.RMSNorm(dim)
        self.up = torch.nn.Linear(dim, 3 * dim, bias=False)
        self.down = torch.nn.Linear(3 * dim, dim, bias=False)
        self.norm2 = torch.nn.RMSNorm(dim)
        self.head = torch.nn.Linear(dim, vocab, bias=False)
        self.head.weight = self.emb.weight

    def forward(self, ids):
        x = self.emb(ids)
        x = x + self.down(torch.nn.functional.silu(self.up(self.norm1(x))))
        return self.head(self.norm2(x))


@pytest.mark.parametrize("max_norm", [0.1, 1.0, 5.0])
def test_clip_matches_torch_on_tied_model(max_norm):
    """torchure tests/grad_helper.py:83-102 restated: clip_grad_norm on a real model
    with a tied embedding vs torch.nn.utils.clip_grad_norm_ (rtol 1e-5, atol 1e-7)."""
    import torchure_amd as ta

    def build():
        torch.manual_seed(0)
        return _TiedLM().to(DEV)

    mine, ref = build(), build()
    g = torch.Generator().manual_seed(1234)
    ids = torch.randint(0, 64, (2, 16), generator=g).to(DEV)
    for m in (mine, ref):
        logits = m(ids)
        loss = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, 64), ids[:, 1:].reshape(-1))
        (loss * 50.0).backward()  # norms large enough that every max_norm clips
    got = ta.clip_grad_norm(mine.parameters(), None, max_norm)
    want = torch.nn.utils.clip_grad_norm_(ref.parameters(), max_norm)
    torch.testing.assert_close(got, want)
    assert len(list(mine.parameters())) == 5  # tied weight counted once
    for (name, p), (_, q) in zip(mine.named_parameters(), ref.named_parameters()):
        torch.testing.assert_close(p.grad, q.grad, rtol=1e-5, atol=1e-7, msg=name)


class _MLPBlockLM(torch.nn.Module):
    """A small pre-norm MLP block with an output head (no embedding, whose backward
    accumulates with atomics and is not bit-reproducible)."""

    def __init__(self, dim=64, vocab=96):
        super().__init__()
        self.norm1 = torch.nn.RMSNorm(dim)
        self.up = torch.nn.Linear(dim, 4 * dim, bias=True)
        self.down = torch.nn.Linear(4 * dim, dim, bias=False)
        self.norm2 = torch.nn.RMSNorm(dim)
        self.head = torch.nn.Linear(dim, vocab, bias=False)

    def forward(self, x):
        h = x + self.down(torch.nn.functional.silu(self.up(self.norm1(x))))
        return self.head(self.norm2(h))


def _train_loop(model, batches, opt, sched, clip, max_norm, micro):
    """torchure/train/trainer.py:370-397 restated: bf16 autocast forward, loss / micro,
    backward (fp32 .grad accumulates over the micro-batches), clip, step, zero_grad,
    scheduler step. Returns the per-step losses and pre-clip norms."""
    losses, norms = [], []
    for step_batches in batches:
        loss = torch.zeros((), device=DEV)
        for x, y in step_batches[:micro]:
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                logits = model(x)
                part = torch.nn.functional.cross_entropy(logits.float().reshape(-1, logits.shape[-1]),
                                                         y.reshape(-1)) / micro
            part.backward()
            loss += part.detach()
        norms.append(clip(model, max_norm).detach().clone())
        opt.step()
        opt.zero_grad()
        sched.step()
        losses.append(loss)
    return torch.stack(losses), torch.stack(norms)


def _run_training(max_norm, steps=6, micro=2, total_steps=6):
    """Runs the same training twice from the same init and data: once through
    torchure_amd (clip_grad_norm + AdamW + WSD schedule), once through the
    reference's torch composition (grad_helper clip, AdamW(fused=True), the WSD
    multiplier through LambdaLR)."""
    import torchure_amd as ta
    from oracle.torch_composition import clip_grad_norm_reference

    g = torch.Generator().manual_seed(99)
    batches = [[(torch.randn(4, 32, 64, generator=g).to(DEV),
                 torch.randint(0, 96, (4, 32), generator=g).to(DEV)) for _ in range(micro)]
               for _ in range(steps)]
    sched_cfg = {"type": "wsd", "total_steps": total_steps, "warmup_ratio": 0.34, "decay_ratio": 0.34}
    hyper = {"lr": 2e-3, "betas": (0.9, 0.95), "eps": 1e-8, "weight_decay": 0.1}

    def build():
        torch.manual_seed(0)
        return _MLPBlockLM().to(DEV)

    def ours():
        model = build()
        opt = ta.build_optimizer(model, "adamw", dict(hyper, fused=True))
        sched = ta.build_scheduler(opt, sched_cfg)
        out = _train_loop(model, batches, opt, sched,
                          lambda m, mn: ta.clip_grad_norm(m.parameters(), None, mn), max_norm, micro)
        return model, opt, out

    def reference():
        model = build()
        params = [p for p in model.parameters() if p.requires_grad]
        groups = [{"params": [p for p in params if p.dim() >= 2], "weight_decay": hyper["weight_decay"]},
                  {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0}]
        opt = torch.optim.AdamW(groups, lr=hyper["lr"], betas=hyper["betas"], eps=hyper["eps"], fused=True)
        sched = torch.optim.lr_scheduler.LambdaLR(
            opt, lambda s: oracle.wsd_scale(s, total_steps, 0.34, 0.34))
        out = _train_loop(model, batches, opt, sched,
                          lambda m, mn: clip_grad_norm_reference([p.grad for p in m.parameters()], mn),
                          max_norm, micro)
        return model, opt, out

    return ours(), reference(), reference


def _assert_reference_reproducible(ref, rerun):
    m2, _, (l2, _) = rerun()
    same = torch.equal(ref[2][0], l2) and all(torch.equal(p, q) for p, q in
                                               zip(ref[0].parameters(), m2.parameters()))
    if not same:
        pytest.skip("torch's own training loop is not bit-reproducible on this box")


def test_training_loop_no_clip_bit_exact_vs_torch():
    """Full loop with a max_norm no step reaches (coefficient 1.0): losses, masters,
    moments and step counters equal torch's fused AdamW loop bit for bit over six
    steps through the whole WSD curve (warmup, stable, decay)."""
    (mine, opt, (loss_a, norm_a)), ref, rerun = _run_training(max_norm=1e9)
    _assert_reference_reproducible(ref, rerun)
    model_r, opt_r, (loss_b, norm_b) = ref
    assert torch.equal(loss_a, loss_b)
    torch.testing.assert_close(norm_a, norm_b, rtol=1e-6, atol=0)
    assert [gr["lr"] for gr in opt.param_groups] == [gr["lr"] for gr in opt_r.param_groups]
    for (name, p), q in zip(mine.named_parameters(), model_r.parameters()):
        assert torch.equal(p, q), name
        sa, sb = opt.state[p], opt_r.state[q]
        assert torch.equal(sa["exp_avg"], sb["exp_avg"]), name
        assert torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"]), name
        assert float(sa["step"]) == float(sb["step"]) == 6.0
        assert p.grad is None


def test_training_loop_with_clip_tracks_torch():
    """Same loop with clipping active on every step. The coefficient comes from this
    library's fp64-accumulated norm and torch's fp32 one, which may differ in the
    last bits, so the trajectories are compared within tolerance: norms to 1e-6
    relative, losses to 1e-5, parameters to rtol 1e-4 / atol 2e-6."""
    (mine, opt, (loss_a, norm_a)), ref, _ = _run_training(max_norm=0.05)
    model_r, opt_r, (loss_b, norm_b) = ref
    assert bool((norm_a > 0.05).all()), norm_a  # every step clipped
    torch.testing.assert_close(norm_a, norm_b, rtol=1e-6, atol=0)
    torch.testing.assert_close(loss_a, loss_b, rtol=1e-5, atol=0)
    for (name, p), q in zip(mine.named_parameters(), model_r.parameters()):
        torch.testing.assert_close(p, q, rtol=1e-4, atol=2e-6, msg=name)


def test_launch_planned_on_one_stream_runs_on_another():
    """A step planned (tables uploaded, workspace allocated) on the default stream and launched
    on a side stream waits for the upload and keeps its buffers alive there: it gives the bits
    of the same step run on one stream. The same for a norm launch."""
    from torchure_amd.core.grad_helper import NormLaunch

    host = H.make_host_set([(300, 200), (1000,), (33,)], seed=44, grad_std=0.01)
    pa, wa, oa = H.device_setup(host, DEV)
    pb, wb, ob = H.device_setup(host, DEV)
    for launch in oa.plan_step():
        launch()
    side = torch.cuda.Stream(device=DEV)
    launches = ob.plan_step()
    norm_a = NormLaunch([w.grad for w in wa], 1.0)
    norm_a()
    norm_b = NormLaunch([w.grad for w in wb], 1.0)
    with torch.cuda.stream(side):
        for launch in launches:
            launch()
        norm_b()
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    for x, y, u, v in zip(pa, pb, wa, wb):
        assert torch.equal(x, y)
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))
        for k in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(oa.state[x][k], ob.state[y][k])
    assert norm_a.norm.view(torch.int32).item() == norm_b.norm.view(torch.int32).item()
    assert norm_a.coef.view(torch.int32).item() == norm_b.coef.view(torch.int32).item()


def test_record_with_unknown_group_is_poisoned():
    """Called through the C ABI with a tensor record whose group index the call does not have,
    tm_adamw_step poisons that tensor instead of stepping it with another group's
    hyper-parameters (its step counter, master, moments become NaN, its bf16 copy 0x7FC0),
    and steps the other records as usual: bit for bit what AdamW.step() gives them."""
    from torchure_amd import _native
    from torchure_amd.core import tables

    host = H.make_host_set([(64, 32), (100,)], seed=81, grad_std=0.01)
    pa, wa, oa = H.device_setup(host, DEV)
    oa.step()  # the reference bits: no clip, the two torchure groups
    pb, wb, ob = H.device_setup(host, DEV)
    rows = np.zeros(2, dtype=_native.TENSOR_DTYPE)
    for i, (p, w) in enumerate(zip(pb, wb)):
        st = ob.state[p]
        rows[i] = (p.data_ptr(), st["exp_avg"].data_ptr(), st["exp_avg_sq"].data_ptr(), w.grad.data_ptr(),
                   w.data_ptr(), st["step"].data_ptr(), p.numel(), 0, _native.TM_GRAD_BF16)
    rows["group"] = [0, 7]
    d_rows = tables.upload(rows, DEV)
    chunk_elems = tables.DEFAULT_CHUNK_ELEMS
    chunks, n_chunks = tables.CHUNKS.get(rows["numel"], chunk_elems, DEV)
    ws = torch.empty(_native.workspace_bytes(2), dtype=torch.uint8, device=DEV)
    hyper = _native.hyper_array([(H.HYPER["lr"], H.HYPER["beta1"], H.HYPER["beta2"], H.WD, H.HYPER["eps"]),
                                 (H.HYPER["lr"], H.HYPER["beta1"], H.HYPER["beta2"], 0.0, H.HYPER["eps"])])
    rc = _native.lib().tm_adamw_step(d_rows.data_ptr(), 2, chunks.data_ptr(), n_chunks, chunk_elems, hyper, 2,
                                     None, ws.data_ptr(), _native.stream_handle(DEV))
    _native.check(rc, "tm_adamw_step")
    torch.cuda.synchronize()
    assert torch.equal(pb[0], pa[0])
    assert torch.equal(wb[0].view(torch.int16), wa[0].view(torch.int16))
    for k in ("step", "exp_avg", "exp_avg_sq"):
        assert torch.equal(ob.state[pb[0]][k], oa.state[pa[0]][k])
    st = ob.state[pb[1]]
    for t in (pb[1], st["step"], st["exp_avg"], st["exp_avg_sq"]):
        assert bool(torch.isnan(t).all())
    assert bool((wb[1].view(torch.int16) == 0x7FC0).all())


def test_chunk_table_built_on_busy_stream_hit_on_another():
    """Chunk tables first built on a side stream whose uploads still wait behind a long kernel,
    then fetched from the cache for a clip + step on another stream: that stream waits for the
    uploads, so the step gives the bits of the same step run on the default stream."""
    import torchure_amd as ta

    shapes = [(1234, 77), (4099,), (55, 3)]  # sizes no other test uses: the first fetch builds
    host = H.make_host_set(shapes, seed=71, grad_std=0.02)
    pa, wa, oa = H.device_setup(host, DEV)
    pb, wb, ob = H.device_setup(host, DEV)
    pc, _, oc = H.device_setup(host, DEV)
    torch.cuda.synchronize()
    busy, other = torch.cuda.Stream(device=DEV), torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(busy):
        torch.cuda._sleep(100_000_000)  # a bounded spin; the table uploads queue behind it
        ta.clip_grad_norm(pc, None, 1.0)
        oc.step()
    with torch.cuda.stream(other):
        ta.clip_grad_norm(pb, None, 1.0)
        ob.step()
    torch.cuda.synchronize()
    ta.clip_grad_norm(pa, None, 1.0)
    oa.step()
    torch.cuda.synchronize()
    for x, y, u, v in zip(pa, pb, wa, wb):
        assert torch.equal(x, y)
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))
        for k in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(oa.state[x][k], ob.state[y][k])


def test_two_optimizers_stepped_from_two_threads():
    """Two optimizers, each clipped and stepped three times from its own host thread on its own
    stream (the library's shared upload buffers are then used concurrently), give the bits of
    the same sequence run on one thread."""
    import threading

    import torchure_amd as ta

    def setup(seed):
        host = H.make_host_set([(256, 128), (777,), (64, 64)], seed=seed, grad_std=0.02)
        return H.device_setup(host, DEV)

    def run(params, opt, stream):
        with torch.cuda.stream(stream):
            norms = []
            for _ in range(3):
                norms.append(ta.clip_grad_norm(params, None, 1.0))
                opt.step()
            return norms

    seq = [setup(50), setup(51)]
    seq_norms = [run(p, o, torch.cuda.current_stream(DEV)) for p, _, o in seq]
    torch.cuda.synchronize()

    thr = [setup(50), setup(51)]
    streams = [torch.cuda.Stream(device=DEV), torch.cuda.Stream(device=DEV)]
    out, errors = [None, None], []

    def worker(i):
        try:
            p, _, o = thr[i]
            out[i] = run(p, o, streams[i])
            streams[i].synchronize()
        except Exception as e:  # reported below
            errors.append(e)

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errors, errors
    torch.cuda.synchronize()
    for (pa, wa, oa), (pb, wb, ob), na, nb in zip(seq, thr, seq_norms, out):
        for x, y, u, v in zip(pa, pb, wa, wb):
            assert torch.equal(x, y)
            assert torch.equal(u.view(torch.int16), v.view(torch.int16))
            for k in ("step", "exp_avg", "exp_avg_sq"):
                assert torch.equal(oa.state[x][k], ob.state[y][k])
        assert [n.view(torch.int32).item() for n in na] == [n.view(torch.int32).item() for n in nb]


def test_stream_copy_copies_every_byte():
    """tm_stream_copy (the bench's streaming-copy ceiling) copies exactly nbytes: sizes that fill
    whole waves and ones that end inside a wave, at buffer offsets of 16 bytes, leaving the bytes
    around the destination range untouched."""
    from torchure_amd import _native

    lib = _native.lib()
    gen = torch.Generator(device=DEV).manual_seed(5)
    src = torch.randint(0, 256, (3 << 20,), dtype=torch.uint8, device=DEV, generator=gen)
    for nbytes, off in ((16, 0), (1024, 16), (1040, 32), (65536 * 16 + 48, 0), ((3 << 20) - 64, 16)):
        dst = torch.full((nbytes + 2 * 64,), 0xA5, dtype=torch.uint8, device=DEV)
        rc = lib.tm_stream_copy(dst.data_ptr() + 64, src.data_ptr() + off, nbytes, _native.stream_handle(DEV))
        _native.check(rc, "tm_stream_copy")
        torch.cuda.synchronize()
        assert torch.equal(dst[64:64 + nbytes], src[off:off + nbytes]), nbytes
        assert bool((dst[:64] == 0xA5).all()) and bool((dst[64 + nbytes:] == 0xA5).all()), nbytes



@pytest.mark.parametrize("chunk_elems", [2048, 10240, 16384, 18432])
def test_fused_and_standalone_norm_partials_bit_equal(chunk_elems):
    """The last micro-step's fused norm and tm_grad_norm over the resulting fp32 buffers form
    the same 2048 fp64 block partials, bit for bit (not only the same fp32 norm): chunks of 8,
    40, 64 and 72 slices (one round of slice partials, a partial round, two rounds), lengths
    around the 256-element slice and the chunk, accumulators that are not 16-byte aligned
    (element-wise lane mapping) and micro-grads that are not 8-byte aligned (the accumulator's
    mapping with 2-byte loads); the sums match fp64 within 1e-12 relative."""
    from torchure_amd import _native

    lib = _native.lib()
    lens = [1, 255, 256, 257, 5000, 16384, 16385, 40000, 100003, 18431]
    acc_off = [0, 64, 1, 128, 3, 0, 2, 64, 0, 5]      # fp32 elements: odd ones break 16 B alignment
    mic_off = [0, 8, 3, 0, 8, 1, 0, 5, 8, 0]          # bf16 elements: odd ones break 8 B alignment
    gen = torch.Generator(device=DEV).manual_seed(99)
    room = sum(lens) + 256 * len(lens)
    acc_pool = torch.randn(room, device=DEV, generator=gen) * 1e-2
    mic_pool = (torch.randn(room, device=DEV, generator=gen) * 2e-3).to(torch.bfloat16)
    accs, mics, pa, pm = [], [], 0, 0
    for n, oa, om in zip(lens, acc_off, mic_off):
        accs.append(acc_pool[pa + oa: pa + oa + n])
        mics.append(mic_pool[pm + om: pm + om + n])
        pa += oa + n + 64 - (oa + n) % 64
        pm += om + n + 64 - (om + n) % 64
    assert [a.numel() for a in accs] == lens and [m.numel() for m in mics] == lens
    numels = np.asarray(lens, dtype=np.int64)
    chunks = torch.from_numpy(_native.fill_chunks(numels, chunk_elems).view(np.uint8).copy()).to(DEV)
    n_chunks = chunks.numel() // 8
    stream = _native.stream_handle(DEV)

    rows = np.zeros(len(lens), dtype=_native.ACCUM_DTYPE)
    rows["acc"] = [a.data_ptr() for a in accs]
    rows["micro"] = [m.data_ptr() for m in mics]
    rows["numel"] = numels
    d_rows = torch.from_numpy(rows.view(np.uint8).copy()).to(DEV)
    ws_a = torch.zeros(int(lib.tm_accum_norm_workspace_bytes(n_chunks, chunk_elems)), dtype=torch.uint8, device=DEV)
    norm_a = torch.empty((), dtype=torch.float32, device=DEV)
    want = [(a.double() + m.double()).float() for a, m in zip(accs, mics)]
    _native.check(lib.tm_grad_accumulate_list(d_rows.data_ptr(), len(lens), chunks.data_ptr(), n_chunks, chunk_elems,
                                              1, ws_a.data_ptr(), ws_a.numel(), norm_a.data_ptr(), stream),
                  "tm_grad_accumulate_list")
    torch.cuda.synchronize()
    for a, w in zip(accs, want):
        assert torch.equal(a.view(torch.int32), w.view(torch.int32))

    trows = np.zeros(len(lens), dtype=_native.TENSOR_DTYPE)
    trows["grad"] = [a.data_ptr() for a in accs]
    trows["numel"] = numels
    trows["flags"] = _native.TM_GRAD_F32
    d_trows = torch.from_numpy(trows.view(np.uint8).copy()).to(DEV)
    ws_b = torch.zeros(_native.workspace_bytes(len(lens)), dtype=torch.uint8, device=DEV)
    norm_b = torch.empty((), dtype=torch.float32, device=DEV)
    _native.check(lib.tm_grad_norm(d_trows.data_ptr(), len(lens), chunks.data_ptr(), n_chunks, chunk_elems, 0.0, 0,
                                   ws_b.data_ptr(), norm_b.data_ptr(), None, stream), "tm_grad_norm")
    torch.cuda.synchronize()
    part_a = ws_a[: 8 * _native.TM_NORM_PARTIALS].view(torch.float64)
    part_b = ws_b[: 8 * _native.TM_NORM_PARTIALS].view(torch.float64)
    assert torch.equal(part_a.view(torch.int64), part_b.view(torch.int64))
    assert norm_a.view(torch.int32).item() == norm_b.view(torch.int32).item()
    exact = math.fsum(float((a.double() ** 2).sum()) for a in accs)
    assert abs(float(part_a.sum()) - exact) <= 1e-12 * exact


@pytest.mark.parametrize("chunk_elems", [None, 2048])
def test_views_off_their_1kib_boundaries_match_oracle(chunk_elems):
    """The update lays each tensor's slices on its fp32 arrays' 1 KiB boundaries, wrapping the
    last elements into the first slice's head. Tensors whose fp32 views start 4 to 252 elements
    past such a boundary, with master, m and v at a shared phase or at different ones, lengths
    that make the wrap take 0, some or all of the head (a whole number of chunks, one element
    past, odd lengths, tensors shorter than the head), an fp32 grad, and a view off 16 bytes
    (element at a time): every element bit for bit against the oracle after a clipped step and
    after a second, unclipped one (the masters are views of one buffer and share one autograd
    version counter, which the working-copy bookkeeping has to follow), and no element outside
    the views written."""
    import torchure_amd as ta

    ce = chunk_elems or 16384
    specs = []
    for ph in (4, 64, 128, 252):
        for n in (1, 3, 5, 100, 252 - ph + 4, 255, 256, 257, ce - ph, ce - ph + 1, ce, ce + 7,
                  3 * ce + 130, 2 * ce - 3, 40003):
            specs.append((n, dict(p=ph, m=ph, v=ph, g=ph, w=ph), False))
    specs += [
        (5 * ce + 77, dict(p=64, m=128, v=128), False),  # m and v agree: their phase
        (5 * ce + 77, dict(p=64, m=64, v=128), False),  # master's phase
        (5 * ce + 77, dict(p=4, m=128, v=252), False),  # all differ: master's phase
        (3 * ce + 11, dict(p=128, m=128, v=128, g=64), True),  # fp32 grad at another phase
        (3 * ce + 11, dict(p=64, m=128, v=128, g=64), True),  # fp32 grad siding with the master
        (2 * ce + 9, dict(p=1, m=1, v=1), False),  # 4 bytes off: element at a time
        (4 * ce, dict(p=0, m=0, v=0), False),  # on the boundary
    ]
    pools, params, work, opt, host = H.views_at_phases(specs, DEV, seed=77, chunk_elems=chunk_elems)
    print(f"phase views: {len(specs)} tensors, chunk_elems {ce}", flush=True)
    norm = ta.clip_grad_norm(params, None, 0.05)
    coef = float(opt._pending[0].item())
    assert coef < 1.0
    opt.step()
    torch.cuda.synchronize()
    tens = H.oracle_tensors(host)
    ref_norm, _ = oracle.reference_step(tens, H.HYPER, 0.05, clip_override=coef)
    assert abs(float(norm.item()) - float(ref_norm)) <= 1e-6 * float(ref_norm)
    w = H.compare_state(params, work, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w
    opt.step()  # same grads, no clip
    torch.cuda.synchronize()
    oracle.reference_step(tens, H.HYPER, None)
    w = H.compare_state(params, work, opt, tens)
    assert w == {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}, w

    # the guards: everything outside the views still holds its sentinel
    for role, pool in pools.items():
        mask = torch.ones(pool.numel(), dtype=torch.bool, device=DEV)
        for i, p in enumerate(params):
            t = {"p": p, "m": opt.state[p]["exp_avg"], "v": opt.state[p]["exp_avg_sq"],
                 "w": work[i], "g": work[i].grad, "gf": p.grad}[role]
            if t is None or t.untyped_storage().data_ptr() != pool.untyped_storage().data_ptr():
                continue
            o = t.storage_offset()
            mask[o: o + t.numel()] = False
        rest = pool[mask]
        if pool.dtype == torch.float32:
            assert torch.isnan(rest).all(), role
        else:
            assert (rest.float() == 7.0).all(), role
