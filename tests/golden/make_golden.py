"""Writes the golden vectors under tests/golden/ from the torch library (CPU).

The reference optimizer step is torch.optim.AdamW(fused=True) (built at
torchure/optimizer/builder.py:46) behind torchure's clip
(torchure/core/grad_helper.py:8-34) and the order of
torchure/train/trainer.py:391-397. torch is a third-party library present
here; the reference's own Python files are not imported. The composition
below calls the same torch functions the reference calls, in the same order:

  norms = torch._foreach_norm(grads, 2.0); total = vector_norm(stack(norms))
  coef  = clamp(max_norm / (total + 1e-6), max=1.0); torch._foreach_mul_(grads, coef)
  torch.optim.AdamW(groups, lr, betas, eps, fused=True).step()
  bf16 working copy = master.to(torch.bfloat16)

Run:  python tests/golden/make_golden.py     (deterministic; seeds fixed)
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

SHAPES = [(64, 48), (33,), (7,), (1,), (130, 17), (4096,), (8, 8), (3, 5)]
HYPER = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()


def make_adamw_case(name: str, seed: int, grad_scale: float, steady: bool, n_steps: int = 3,
                    max_norm: float | None = 1.0) -> None:
    rng = np.random.Generator(np.random.PCG64(seed))
    p0, m0, v0, gs = [], [], [], []
    for s in SHAPES:
        n = int(np.prod(s))
        p0.append((rng.standard_normal(n) * 0.02).astype(np.float32).reshape(s))
        if steady:
            m0.append((rng.standard_normal(n) * 1e-4).astype(np.float32).reshape(s))
            v0.append((np.abs(rng.standard_normal(n)) * 1e-8).astype(np.float32).reshape(s))
        else:
            m0.append(np.zeros(s, np.float32))
            v0.append(np.zeros(s, np.float32))
        gs.append([bf16_round((rng.standard_normal(n) * grad_scale).astype(np.float32)).reshape(s)
                   for _ in range(n_steps)])
    # a tensor whose grad is all zero in every step (still updated)
    gs[2] = [np.zeros(SHAPES[2], np.float32) for _ in range(n_steps)]
    step0 = 1000.0 if steady else 0.0

    params = [torch.nn.Parameter(torch.from_numpy(p.copy())) for p in p0]
    groups = [
        {"params": [p for p in params if p.dim() >= 2], "weight_decay": HYPER["weight_decay"]},
        {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0},
    ]
    opt = torch.optim.AdamW(groups, lr=HYPER["lr"], betas=HYPER["betas"], eps=HYPER["eps"], fused=True)
    if steady or step0:
        for p, m, v in zip(params, m0, v0):
            opt.state[p]["step"] = torch.tensor(step0, dtype=torch.float32)
            opt.state[p]["exp_avg"] = torch.from_numpy(m.copy())
            opt.state[p]["exp_avg_sq"] = torch.from_numpy(v.copy())
    out = {"shapes": np.array([str(s) for s in SHAPES]), "step0": np.float32(step0),
           "lr": np.float64(HYPER["lr"]), "beta1": np.float64(HYPER["betas"][0]),
           "beta2": np.float64(HYPER["betas"][1]), "eps": np.float64(HYPER["eps"]),
           "weight_decay": np.float64(HYPER["weight_decay"]),
           "max_norm": np.float32(np.nan if max_norm is None else max_norm)}
    for i in range(len(SHAPES)):
        out[f"p0_{i}"] = p0[i]
        out[f"m0_{i}"] = m0[i]
        out[f"v0_{i}"] = v0[i]
    for k in range(n_steps):
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(gs[i][k].copy())
            out[f"g{k}_{i}"] = gs[i][k]
        grads = [p.grad for p in params]
        norms = torch._foreach_norm(grads, 2.0)
        total = torch.linalg.vector_norm(torch.stack(norms), 2.0)
        out[f"norm{k}"] = np.float32(total.item())
        if max_norm is not None:
            coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
            torch._foreach_mul_(grads, coef)
            out[f"coef{k}"] = np.float32(coef.item())
        opt.step()
        for i, p in enumerate(params):
            st = opt.state[p]
            out[f"p{k + 1}_{i}"] = p.detach().numpy().copy()
            out[f"m{k + 1}_{i}"] = st["exp_avg"].numpy().copy()
            out[f"v{k + 1}_{i}"] = st["exp_avg_sq"].numpy().copy()
            out[f"bf{k + 1}_{i}"] = p.detach().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
            out[f"step{k + 1}_{i}"] = np.float32(st["step"].item())
        opt.zero_grad()
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


def make_bf16_case() -> None:
    special = np.array([
        0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, -np.nan,
        1.0 + 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9,
        np.float32(3.4028235e38), 1e-40, -1e-40, 1.17549435e-38, 2 ** -133, 65504.0, 0.1, -0.3,
    ], dtype=np.float32)
    ties = (np.arange(1, 257, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    rng = np.random.Generator(np.random.PCG64(7))
    rand = rng.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([special, ties, rand]).astype(np.float32)
    bits = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(os.path.join(HERE, "bf16_rne.npz"), x=x, bits=bits)


def main() -> None:
    torch.set_num_threads(1)
    make_adamw_case("adamw_fresh_noclip", seed=11, grad_scale=1e-3, steady=False, max_norm=1.0)
    make_adamw_case("adamw_steady_clip", seed=12, grad_scale=0.1, steady=True, max_norm=1.0)
    make_adamw_case("adamw_steady_measure", seed=13, grad_scale=1e-3, steady=True, max_norm=None)
    make_bf16_case()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
