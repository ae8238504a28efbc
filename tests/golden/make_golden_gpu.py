"""Writes golden vectors of torch-ROCm's own GPU kernels (run on an MI355X).

  adamw_rocm_fused.npz  inputs and outputs of torch._fused_adamw_ (reached via
                        torch.optim.AdamW(fused=True), the optimizer torchure builds at
                        torchure/optimizer/builder.py:46) for several value regimes
  bf16_rne_rocm.npz     torch's device fp32 -> bf16 cast of the bf16_rne.npz inputs

These pin the oracle's GPU recipe bit for bit (tests/test_oracle.py). Usage:
  python tests/golden/make_golden_gpu.py OUTDIR      (then copy the .npz files here)
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def adamw_cases(dev):
    rng = np.random.Generator(np.random.PCG64(2024))
    n = 4096
    cases = []
    # (name, step_before, p_std, m_std, v_scale, g_std, wd)
    regimes = [
        ("fresh", 0.0, 0.02, 0.0, 0.0, 1e-3, 0.1),
        ("steady", 1000.0, 0.02, 1e-4, 1e-8, 1e-3, 0.1),
        ("steady_nodecay", 1000.0, 0.02, 1e-4, 1e-8, 1e-3, 0.0),
        ("decay_phase", 9800.0, 0.05, 1e-3, 1e-6, 2e-2, 0.1),
        ("tiny_v", 3.0, 0.02, 1e-6, 1e-20, 1e-9, 0.1),
        ("large", 10.0, 3.0, 1.0, 1.0, 5.0, 0.1),
        ("zero_grad", 500.0, 0.02, 1e-4, 1e-8, 0.0, 0.1),
    ]
    lr, b1, b2, eps = 3e-4, 0.9, 0.95, 1e-8
    out = {"lr": np.float64(lr), "beta1": np.float64(b1), "beta2": np.float64(b2), "eps": np.float64(eps)}
    for k, (name, step0, ps, ms, vs, gs, wd) in enumerate(regimes):
        p = (rng.standard_normal(n) * ps).astype(np.float32)
        m = (rng.standard_normal(n) * ms).astype(np.float32)
        v = (np.abs(rng.standard_normal(n)) * vs).astype(np.float32)
        g = (rng.standard_normal(n) * gs).astype(np.float32)
        par = torch.nn.Parameter(torch.from_numpy(p.copy()).to(dev))
        opt = torch.optim.AdamW([par], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd, fused=True)
        par.grad = torch.from_numpy(g.copy()).to(dev)
        st = opt.state[par]
        st["step"] = torch.tensor(step0, dtype=torch.float32, device=dev)
        st["exp_avg"] = torch.from_numpy(m.copy()).to(dev)
        st["exp_avg_sq"] = torch.from_numpy(v.copy()).to(dev)
        opt.step()
        torch.cuda.synchronize()
        out[f"name{k}"] = np.array(name)
        out[f"p_in{k}"], out[f"m_in{k}"], out[f"v_in{k}"], out[f"g{k}"] = p, m, v, g
        out[f"wd{k}"] = np.float64(wd)
        out[f"step_after{k}"] = np.float32(st["step"].item())
        out[f"p_out{k}"] = par.detach().cpu().numpy()
        out[f"m_out{k}"] = st["exp_avg"].cpu().numpy()
        out[f"v_out{k}"] = st["exp_avg_sq"].cpu().numpy()
    out["n_cases"] = np.int64(len(regimes))
    return out


def main(outdir: str) -> None:
    dev = torch.device("cuda:0")
    os.makedirs(outdir, exist_ok=True)
    np.savez_compressed(os.path.join(outdir, "adamw_rocm_fused.npz"), **adamw_cases(dev))
    z = np.load(os.path.join(HERE, "bf16_rne.npz"), allow_pickle=False)
    x = z["x"]
    bits = torch.from_numpy(x.copy()).to(dev).to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    np.savez_compressed(os.path.join(outdir, "bf16_rne_rocm.npz"), x=x, bits=bits)
    print("wrote", outdir)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else HERE)
