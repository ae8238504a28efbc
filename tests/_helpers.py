"""Shared helpers of the parity tests: seeded param sets, ulp distances, oracle runs."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle

HYPER = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8)
WD = 0.1


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def ulp_diff(a, b) -> np.ndarray:
    """|a - b| in units of fp32 ulp (ordered-integer distance; +-0 are 0 apart)."""
    ai = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    bi = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def make_host_set(shapes, seed, *, steady=True, grad_std=1e-3, zero_grad_every=0, grad_dtype="bf16",
                  step0=None):
    """numpy state for a param list: p ~ N(0,.02), m ~ N(0,1e-4), v = |N(0,1)|*1e-8."""
    r = rng(seed)
    out = []
    for i, s in enumerate(shapes):
        n = int(np.prod(s))
        p = (r.standard_normal(n) * 0.02).astype(np.float32)
        if steady:
            m = (r.standard_normal(n) * 1e-4).astype(np.float32)
            v = (np.abs(r.standard_normal(n)) * 1e-8).astype(np.float32)
        else:
            m = np.zeros(n, np.float32)
            v = np.zeros(n, np.float32)
        g = (r.standard_normal(n) * grad_std).astype(np.float32)
        if zero_grad_every and i % zero_grad_every == zero_grad_every - 1:
            g[:] = 0
        gb = oracle.bf16_rne(g)
        out.append(dict(shape=tuple(s), p=p, m=m, v=v,
                        g=gb if grad_dtype == "bf16" else oracle.bf16_to_f32(gb).copy(),
                        step=(1000.0 if steady else 0.0) if step0 is None else float(step0),
                        wd=WD if len(s) >= 2 else 0.0, out=np.zeros(n, np.uint16)))
    return out


def to_dev_bf16(bits: np.ndarray, shape, dev) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).view(shape).to(dev)


def from_dev_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def device_setup(host, dev, *, working=True, grad_on_master=False):
    """Build fp32 masters (+ bf16 working copies with grads) and an AdamW with the
    torchure param groups; state primed from ``host``."""
    import torchure_amd as ta

    params = [torch.nn.Parameter(torch.from_numpy(h["p"].copy()).view(h["shape"]).to(dev)) for h in host]
    work = ta.attach_bf16_working_params(params) if working else None
    for i, h in enumerate(host):
        if grad_on_master or h["g"].dtype == np.float32:
            g = h["g"] if h["g"].dtype == np.float32 else oracle.bf16_to_f32(h["g"])
            params[i].grad = torch.from_numpy(g.copy()).view(h["shape"]).to(dev)
        else:
            work[i].grad = to_dev_bf16(h["g"], h["shape"], dev)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": HYPER["lr"], "weight_decay": WD,
                              "betas": (HYPER["beta1"], HYPER["beta2"]), "fused": True})
    opt.init_state()  # the optimizer's own (pooled) layout, filled in place below
    for p, h in zip(params, host):
        st = opt.state[p]
        if st:
            st["step"].fill_(float(h["step"]))
            st["exp_avg"].copy_(torch.from_numpy(h["m"].copy()).view(h["shape"]))
            st["exp_avg_sq"].copy_(torch.from_numpy(h["v"].copy()).view(h["shape"]))
        else:  # no grad, so no lazy state: primed as separate tensors
            st["step"] = torch.tensor(h["step"], dtype=torch.float32, device=dev)
            st["exp_avg"] = torch.from_numpy(h["m"].copy()).view(h["shape"]).to(dev)
            st["exp_avg_sq"] = torch.from_numpy(h["v"].copy()).view(h["shape"]).to(dev)
    return params, work, opt


def oracle_tensors(host):
    return [dict(p=h["p"].copy(), m=h["m"].copy(), v=h["v"].copy(), g=h["g"], step=h["step"],
                 wd=h["wd"], out=np.zeros(h["p"].size, np.uint16)) for h in host]


def compare_state(params, work, opt, tens, *, max_ulp=0):
    """Max ulp distance of master/m/v and bf16 mismatches between device and oracle."""
    worst = {"p": 0, "m": 0, "v": 0, "bf16": 0, "step": 0}
    for i, (p, t) in enumerate(zip(params, tens)):
        st = opt.state[p]
        worst["p"] = max(worst["p"], int(ulp_diff(p.detach().cpu().numpy().reshape(-1), t["p"]).max(initial=0)))
        worst["m"] = max(worst["m"], int(ulp_diff(st["exp_avg"].cpu().numpy().reshape(-1), t["m"]).max(initial=0)))
        worst["v"] = max(worst["v"], int(ulp_diff(st["exp_avg_sq"].cpu().numpy().reshape(-1), t["v"]).max(initial=0)))
        if work is not None:
            worst["bf16"] += int((from_dev_bf16(work[i]) != t["out"]).sum())
        worst["step"] = max(worst["step"], abs(float(st["step"].item()) - t["step"]))
    return worst


def views_at_phases(specs, dev, seed, chunk_elems=None):
    """Tensors as views of one pool per role (master, m, v fp32; grad and working copy bf16, or
    an fp32 grad on the master), each placed so that its fp32 views start the given number of
    elements past a 1 KiB boundary. ``specs``: (numel, {role: elements past 1 KiB}, fp32 grad).
    Every view is surrounded by guard elements holding a sentinel. Returns the pools, the views
    and the host state."""
    import torchure_amd as ta
    from torchure_amd.optimizer.working import mark_current

    host = make_host_set([(n,) for n, _, _ in specs], seed=seed)
    for h, (_, _, f32) in zip(host, specs):
        h["wd"] = WD  # every view is stepped in the decay group (one-element tensors included)
        if f32:
            h["g"] = oracle.bf16_to_f32(h["g"]).copy()
    gap = 1024  # guard elements between views (a multiple of 256)
    offs, total = [], gap
    for n, _, _ in specs:
        offs.append(total)
        total += (n + 256 + gap + 255) // 256 * 256
    pools = {r: torch.full((total,), float("nan"), device=dev) for r in ("p", "m", "v", "gf")}
    pools["g"] = torch.full((total,), 7.0, device=dev).to(torch.bfloat16)
    pools["w"] = torch.full((total,), 7.0, device=dev).to(torch.bfloat16)

    def view(role, i, n, lead):
        pool = pools[role]
        base = pool.data_ptr() // pool.element_size()
        shift = (lead - (base + offs[i])) % 256 if role in ("p", "m", "v", "gf") else lead
        return pool[offs[i] + shift: offs[i] + shift + n]

    params, work, grads = [], [], []
    for i, ((n, leads, f32), h) in enumerate(zip(specs, host)):
        pv = view("p", i, n, leads.get("p", 0))
        pv.copy_(torch.from_numpy(h["p"]))
        p = torch.nn.Parameter(pv)
        w = view("w", i, n, leads.get("w", 0))
        w.copy_(pv.to(torch.bfloat16))
        p._tm_working = w
        if f32:
            g = view("gf", i, n, leads.get("g", 0))
            g.copy_(torch.from_numpy(h["g"]))
            p.grad = g
        else:
            g = view("g", i, n, leads.get("g", 0))
            g.copy_(to_dev_bf16(h["g"], (n,), dev))
            w.grad = g
        params.append(p)
        work.append(w)
    opt = ta.AdamW([{"params": params, "weight_decay": WD}], lr=HYPER["lr"],
                   betas=(HYPER["beta1"], HYPER["beta2"]), fused=True,
                   **({"chunk_elems": chunk_elems} if chunk_elems else {}))
    for i, ((n, leads, _), p, h) in enumerate(zip(specs, params, host)):
        st = opt.state[p]
        st["step"] = torch.tensor(h["step"], dtype=torch.float32, device=dev)
        st["exp_avg"] = view("m", i, n, leads.get("m", 0))
        st["exp_avg"].copy_(torch.from_numpy(h["m"]))
        st["exp_avg_sq"] = view("v", i, n, leads.get("v", 0))
        st["exp_avg_sq"].copy_(torch.from_numpy(h["v"]))
    # views of one pool share one autograd version counter: mark the copies current only
    # after the last write into the pools
    for p, w in zip(params, work):
        mark_current(p, w)
    torch.cuda.synchronize()
    return pools, params, work, opt, host
