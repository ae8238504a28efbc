"""Benchmark of the MI355X optimizer step (clip + fused AdamW + bf16 refresh).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen3-4b|qwen3-0.6b|...]

One "step" = clip_grad_norm (two-pass norm) + AdamW.step() (step counters,
fused update, bf16 working copies) over the whole parameter set, through the
package's public API, with every tensor already resident in HBM. Inputs are
synthetic (the 4B steady-state configuration: master ~ N(0, .02),
m ~ N(0, 1e-4), v = |N(0,1)| * 1e-8, bf16 grads ~ N(0, 1e-3), step 1000,
lr 3e-4, betas (0.9, 0.95), wd 0.1 on >=2-D, clip 1.0).

Prints one JSON line. ``value`` is whole-step throughput in GB/s of
algorithmic traffic (30 B/param: 2 for the norm pass, 28 for the update);
``roofline`` is for the dominant kernel (the fused update, 28 B/param), timed
with events on the stream it runs on; ``cpu_baseline`` times the reference
composition (torch CPU: foreach-norm clip + torch.optim.AdamW(fused=True) +
bf16 cast) on a bounded sample of the same parameter set on the host cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
UPDATE_BYTES_PER_PARAM = 28  # grad 2 + master/m/v 12 read; master/m/v 12 + bf16 2 written
NORM_BYTES_PER_PARAM = 2
STEP_BYTES_PER_PARAM = UPDATE_BYTES_PER_PARAM + NORM_BYTES_PER_PARAM


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="qwen3-4b")
    ap.add_argument("--chunk-elems", type=int, default=None)
    ap.add_argument("--alloc-conf", default="expandable_segments:True",
                    help="PYTORCH_CUDA_ALLOC_CONF for the run, set before torch starts; the default is "
                         "the reference trainer's own setting (torchure/train/trainer.py:39); '' keeps "
                         "the environment's")
    ap.add_argument("--cpu-configs", default="qwen3-4b,qwen3-0.6b,qwen3-0.6b-ref",
                    help="full parameter sets timed for the CPU baseline; the first is the headline "
                         "(empty = skip)")
    ap.add_argument("--cpu-steps", type=int, default=3, help="at least this many timed CPU steps per set")
    ap.add_argument("--cpu-seconds", type=float, default=4.0,
                    help="keep timing CPU steps of a set until this much CPU work has been timed "
                         "(at most 100 steps)")
    ap.add_argument("--also", default="qwen3-4b-again,qwen3-0.6b,qwen3-0.6b-ref,qwen3-0.6b-fp32acc,"
                                      "qwen3-4b-dropin,qwen3-4b-ddpbuckets,qwen3-4b-eager,ragged,"
                                      "qwen3-4b-shard8",
                    help="comma list of extra configs reported under 'extra' (empty = none); "
                         "'<config>-again' runs that config once more, on fresh allocations made "
                         "after the earlier legs' memory was released; '<config>-eager' steps with "
                         "the clip scaling the grads in place first (defer_clip=False); "
                         "'<config>-shard<N>' steps rank 0's share of that set sharded on dim 0 over "
                         "N ranks (one GPU's part of a sharded step; its norm is the rank's partial)")
    ap.add_argument("--mode", choices=("bench", "kernels", "ce", "ce-gemm"), default="bench",
                    help="kernels: only the norm and update launches (for an -fp32acc config, the "
                         "accumulation launches), --reps times each, plus a 2 GiB device copy for "
                         "calibrating HBM byte counters (for rocprofv3 --pmc); ce: the fused linear "
                         "+ CE legs only; ce-gemm: the fused CE's grad_h GEMM, split-K kernel and "
                         "torch.matmul, at --gemm-shapes")
    ap.add_argument("--ce-dim", type=int, default=1024,
                    help="ce mode: hidden size of the head (1024: Qwen3-0.6B, 2560: Qwen3-4B)")
    ap.add_argument("--gemm-shapes", default="1024x1024,4096x1024,8192x1024,1024x2560,4096x2560",
                    help="ce-gemm mode: comma list of ROWSxDIM grad_h shapes (vocabulary 151,936)")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--states", type=int, default=1,
                    help="kernels mode: build this many copies of the state, each its own set of "
                         "allocations held at once, and launch the norm and update on each in turn "
                         "(placement in HBM differs between them)")
    ap.add_argument("--state-layouts", default="",
                    help="kernels mode: comma list of state layouts built in this order and held at "
                         "once: 'sep' (every tensor its own allocation), 'pool' (one allocation per "
                         "role, tensors are views), 'mv' (separate masters and grads, exp_avg and "
                         "exp_avg_sq pooled); overrides --states")
    ap.add_argument("--fused-ce", type=int, default=1,
                    help="also time the chunked fused linear + CE on the Qwen3-0.6B head (1 = yes)")
    ap.add_argument("--torch-reference", type=int, default=1,
                    help="also time torch-ROCm's own GPU path (foreach clip + fused AdamW) on the "
                         "same config and device (1 = yes)")
    return ap.parse_args()


def run_kernels_only(config: str, reps: int, chunk_elems, dev, states: int = 1, layouts=()):
    """Launch sequence profiled by rocprofv3 --pmc: `reps` x (norm, update), then a
    plain copy of 2 GiB (512 Mi fp32) whose FETCH_SIZE/WRITE_SIZE calibrate the counters.
    For an ``-fp32acc`` config: `reps` x a middle micro-step's accumulation
    (accumulate_list_kernel), then `reps` x the last micro-step's (accumulate_list_sumsq_kernel,
    slice_reduce_kernel, norm_finalize_kernel).
    The state is built from a few pooled buffers (every tensor a view), so setting it up
    takes a handful of device dispatches however many tensors the config has."""
    import torch

    from torchure_amd.core.grad_helper import NormLaunch

    acc_cfg = config.endswith("-fp32acc")
    base = config[: -len("-fp32acc")] if acc_cfg else config
    if (states > 1 or layouts) and not acc_cfg:
        layouts = list(layouts) or ["pool"] * states
        sets = [build_state(base, chunk_elems, dev, pooled=(lay == "pool"), pooled_state=(lay == "mv"))
                for lay in layouts]
        times = []
        for params, work, opt, n_params in sets:
            norm_l = NormLaunch([w.grad for w in work], 1.0)
            norm_l()
            upd = opt.plan_step(norm_l.coef, {id(p) for p in params})
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            for _ in range(reps):
                norm_l()
                a.record()
                upd[0]()
                b.record()
            torch.cuda.synchronize()
            times.append(round(a.elapsed_time(b), 3))
            del upd, norm_l
        print(json.dumps({"mode": "kernels", "config": config, "layouts": layouts,
                          "last_update_ms_per_state": times}), flush=True)
        del sets, params, work, opt
        torch.cuda.empty_cache()
        return
    params, work, opt, n_params = build_state(base, chunk_elems, dev, pooled=True)
    if acc_cfg:
        from torchure_amd.optimizer.working import accumulate_grads_

        micro = [w.grad for w in work]
        accumulate_grads_(params)  # first micro-step: assigns the fp32 accumulators
        for _ in range(reps):
            for w, m in zip(work, micro):
                w.grad = m
            accumulate_grads_(params)
        for _ in range(reps):
            for w, m in zip(work, micro):
                w.grad = m
            accumulate_grads_(params, last=True)
        torch.cuda.synchronize()
        del micro
    else:
        norm_l = NormLaunch([w.grad for w in work], 1.0)
        norm_l()
        upd = opt.plan_step(norm_l.coef, {id(p) for p in params})
        for _ in range(reps):
            norm_l()
            upd[0]()
        torch.cuda.synchronize()
        del upd, norm_l
    del params, work, opt
    torch.cuda.empty_cache()
    a = torch.ones(512 * 1024 * 1024, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    out = {"mode": "kernels", "config": config, "params": n_params, "reps": reps,
           "copy_bytes_each_way": a.numel() * 4}
    if acc_cfg:
        out["accumulate_algorithmic_bytes"] = n_params * 10  # read bf16 2 + fp32 4, write fp32 4
    else:
        out["update_algorithmic_bytes"] = n_params * UPDATE_BYTES_PER_PARAM
        out["norm_algorithmic_bytes"] = n_params * NORM_BYTES_PER_PARAM
    print(json.dumps(out), flush=True)


def build_state(config: str, chunk_elems, dev, pooled: bool = False, pooled_state: bool = False):
    """The steady-state inputs, allocated in the trainer's order: the fp32 masters (the
    model), their bf16 working copies, the grads (backward), then the optimizer state, created
    by the optimizer as its first step creates it (``AdamW.init_state``: pooled moments) and
    filled in place with the steady-state values. With ``pooled`` every role is one buffer
    filled by one random draw and the tensors are views of it; with ``pooled_state`` the
    moments are views of two pools made here (layout experiments)."""
    import torch

    import torchure_amd as ta
    from torchure_amd.core import tables
    from torchure_amd.workloads import shapes_for

    shapes = shapes_for(config)
    g = torch.Generator(device=dev).manual_seed(1234)
    sizes = [math.prod(s) for s in shapes]
    offs = [0]
    for k in sizes:
        offs.append(offs[-1] + (k + 63) // 64 * 64)  # 256-byte aligned views

    def pool(scale, dtype=torch.float32, absval=False):
        flat = torch.randn(offs[-1], device=dev, generator=g).mul_(scale)
        if absval:
            flat.abs_()
        flat = flat.to(dtype)
        return [flat[o: o + k].view(s) for o, k, s in zip(offs, sizes, shapes)]

    if pooled:
        params = [torch.nn.Parameter(t) for t in pool(0.02)]
        work = ta.attach_bf16_working_params(params)
        for w, t in zip(work, pool(1e-3, torch.bfloat16)):
            w.grad = t
    else:
        params = [torch.nn.Parameter(torch.randn(s, device=dev, generator=g) * 0.02) for s in shapes]
        work = ta.attach_bf16_working_params(params)
        for w in work:
            w.grad = (torch.randn(w.shape, device=dev, generator=g) * 1e-3).to(torch.bfloat16)
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True,
                              "chunk_elems": chunk_elems or tables.DEFAULT_CHUNK_ELEMS})
    ms = pool(1e-4) if pooled or pooled_state else None
    vs = pool(1e-8, absval=True) if pooled or pooled_state else None
    steps = torch.full((len(params),), 1000.0, dtype=torch.float32, device=dev) if pooled else None
    for i, p in enumerate(params):
        st = opt.state[p]
        if pooled:
            st["step"], st["exp_avg"], st["exp_avg_sq"] = steps[i], ms[i], vs[i]
        elif pooled_state:
            st["step"] = torch.tensor(1000.0, dtype=torch.float32, device=dev)
            st["exp_avg"], st["exp_avg_sq"] = ms[i], vs[i]
        else:
            if not st:
                opt.init_state()
                st = opt.state[p]
            st["step"].fill_(1000.0)
            st["exp_avg"].copy_(torch.randn(p.shape, device=dev, generator=g) * 1e-4)
            st["exp_avg_sq"].copy_(torch.randn(p.shape, device=dev, generator=g).abs_() * 1e-8)
    torch.cuda.synchronize()
    n_params = sum(p.numel() for p in params)
    return params, work, opt, n_params


def run_gpu(config: str, steps: int, warmup: int, chunk_elems, dev):
    import torch

    import torchure_amd as ta

    params, work, opt, n_params = build_state(config, chunk_elems, dev)
    stream = torch.cuda.current_stream(dev)

    def one_step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        ta.clip_grad_norm(params, None, 1.0)
        if ev is not None:
            ev[1].record(stream)
        opt.step()
        if ev is not None:
            ev[2].record(stream)

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        one_step(evs[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ev_ms = [e[0].elapsed_time(e[2]) for e in evs]

    # Kernel timing: the same launches back to back, bracketed by events on the
    # stream they run on, so host-side work never shows up as device time.
    from torchure_amd.core.grad_helper import NormLaunch

    norm_l = NormLaunch([w.grad for w in work], 1.0)
    norm_l()
    upd = opt.plan_step(norm_l.coef, {id(p) for p in params})  # clip fused, as in a step
    assert len(upd) == 1
    reps = max(5, min(steps, 50))
    a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        norm_l()
    b.record(stream)
    for _ in range(reps):
        upd[0]()
    c.record(stream)
    torch.cuda.synchronize()
    norm_ms = [a.elapsed_time(b) / reps]
    upd_ms = [b.elapsed_time(c) / reps]
    del upd, norm_l
    # Ceiling reference for a 1:1 read/write stream on this device: 4 GiB copied by
    # tm_stream_copy (the library's best streaming copy shape) and by torch's own
    # device-to-device copy, same event timing (reads 4 GiB, writes 4 GiB).
    src = torch.ones(1024 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    lib = ta._native.lib()

    def lib_copy():
        ta._native.check(lib.tm_stream_copy(dst.data_ptr(), src.data_ptr(), src.numel() * 4,
                                            ta._native.stream_handle(dev)), "tm_stream_copy")

    copy_gbps = {}
    for name, fn in (("stream_copy", lib_copy), ("torch_copy", lambda: dst.copy_(src))):
        fn()
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(5):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        copy_gbps[name] = 2 * src.numel() * 4 / (a.elapsed_time(b) / 5 * 1e-3) / 1e9
    del src, dst
    out = dict(
        config=config,
        n_params=n_params,
        n_tensors=len(params),
        ms_per_step=wall * 1e3 / steps,
        ms_per_step_events_median=statistics.median(step_ev_ms),
        norm_ms_mean=statistics.fmean(norm_ms),
        update_ms_mean=statistics.fmean(upd_ms),
        kernel_reps=reps,
        copy_GBps=round(copy_gbps["stream_copy"], 1),
        torch_copy_GBps=round(copy_gbps["torch_copy"], 1),
    )
    del params, work, opt
    torch.cuda.empty_cache()
    return out


def run_gpu_eager(config: str, steps: int, warmup: int, chunk_elems, dev):
    """The reference's own clip order with the optimizer built with ``defer_clip=False``:
    clip_grad_norm scales the bf16 grads in place (torchure/core/grad_helper.py:33, the
    eager scale kernel: read 2 + write 2 B/param), then AdamW.step() reads the scaled grads.
    34 B/param a step (norm 2 + scale 4 + update 28), against 30 with the clip deferred into
    the update. Also times the scale launch alone, back to back, with events."""
    import torch

    import torchure_amd as ta
    from torchure_amd.core.grad_helper import scale_grads_

    params, work, opt, n_params = build_state(config, chunk_elems, dev)
    opt.defer_clip = False
    stream = torch.cuda.current_stream(dev)

    def one():
        ta.clip_grad_norm(params, None, 1.0)
        opt.step()

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    grads = [w.grad for w in work]
    coef = torch.tensor(1.0, dtype=torch.float32, device=dev)  # a multiply by 1.0 keeps the grads
    scale_grads_(grads, coef)
    reps = max(5, min(steps, 50))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        scale_grads_(grads, coef)
    b.record(stream)
    torch.cuda.synchronize()
    scale_ms = a.elapsed_time(b) / reps
    del params, work, opt, grads
    torch.cuda.empty_cache()
    gbs = 34 * n_params / (ms * 1e-3) / 1e9
    return dict(config=config + "-eager-clip", n_params=n_params, ms_per_step=round(ms, 4), bytes_per_param=34,
                GBps=round(gbs, 1), frac_of_peak=round(gbs / PEAK_HBM_GBS, 4), scale_ms_mean=round(scale_ms, 4),
                scale_GBps=round(4 * n_params / (scale_ms * 1e-3) / 1e9, 1))


def ddp_bucket_grads(params, bucket_mb: int = 25) -> int:
    """Gives ``params`` fp32 grads laid out as torchure's DDP leaves them after a sync
    (torchure/parallelism/data_parallel.py:53-66,86-105,120-130): buckets in reverse
    parameter order, closed before a param that would push them past ``bucket_mb`` MiB; a
    bucket of several params is one flat buffer and each ``.grad`` is a view of it, a
    bucket of one param keeps that param's own grad tensor. Returns the bucket count."""
    import torch

    cap = bucket_mb * 1024 * 1024
    runs, run, run_bytes = [], [], 0
    for p in reversed(params):
        nb = p.numel() * p.element_size()
        if run and run_bytes + nb > cap:
            runs.append(run)
            run, run_bytes = [], 0
        run.append(p)
        run_bytes += nb
    if run:
        runs.append(run)
    for run in runs:
        if len(run) == 1:
            continue
        flat = torch.empty(sum(p.numel() for p in run), dtype=torch.float32, device=run[0].device)
        off = 0
        for p in run:
            view = flat[off: off + p.numel()].view_as(p)
            view.copy_(p.grad)
            p.grad = view
            off += p.numel()
    return len(runs)


def run_gpu_dropin(config: str, steps: int, warmup: int, chunk_elems, dev, buckets: bool = False):
    """The plain drop-in configuration: fp32 masters with fp32 .grad (what autograd
    leaves when the model trains on fp32 params under autocast, as the reference's
    trainer does), no bf16 working copies. One step = clip_grad_norm (norm pass,
    4 B/param) + AdamW.step() with the clip fused (28 B/param: read g/p/m/v, write
    p/m/v) = 32 B/param. With ``buckets`` the grads are views into DDP's flat bucket
    buffers (``ddp_bucket_grads``), the layout the step reads after a multi-GPU sync."""
    import torch

    import torchure_amd as ta
    from torchure_amd.core import tables
    from torchure_amd.workloads import shapes_for

    shapes = shapes_for(config)
    g = torch.Generator(device=dev).manual_seed(2468)
    params = [torch.nn.Parameter(torch.randn(s, device=dev, generator=g) * 0.02) for s in shapes]
    for p in params:
        p.grad = torch.randn(p.shape, device=dev, generator=g) * 1e-3
    n_buckets = ddp_bucket_grads(params) if buckets else None
    opt = ta.build_optimizer(torch.nn.ParameterList(params), "adamw",
                             {"lr": 3e-4, "weight_decay": 0.1, "betas": (0.9, 0.95), "fused": True,
                              "chunk_elems": chunk_elems or tables.DEFAULT_CHUNK_ELEMS})
    opt.init_state()  # the optimizer's own (pooled) state, filled in place
    for p in params:
        st = opt.state[p]
        st["step"].fill_(1000.0)
        st["exp_avg"].copy_(torch.randn(p.shape, device=dev, generator=g) * 1e-4)
        st["exp_avg_sq"].copy_(torch.randn(p.shape, device=dev, generator=g).abs_() * 1e-8)

    def one():
        ta.clip_grad_norm(params, None, 1.0)
        opt.step()

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    n = sum(p.numel() for p in params)
    del params, opt
    torch.cuda.empty_cache()
    out = dict(config=config + ("-ddp-buckets-fp32grads" if buckets else "-dropin-fp32grads"), n_params=n,
               ms_per_step=round(ms, 4), bytes_per_param=32, GBps=round(32 * n / (ms * 1e-3) / 1e9, 1),
               frac_of_peak=round(32 * n / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
    if buckets:
        out["ddp_buckets_25MiB"] = n_buckets
    return out


def run_gpu_fp32acc(config: str, steps: int, warmup: int, chunk_elems, dev):
    """Config-3 style step: bf16 micro-grads accumulated into fp32 .grad; the last
    micro-step's accumulation also yields the global norm (fused), clip_grad_norm
    reuses it, and the step reads fp32 grads. Per iteration: last micro-step
    accumulate+norm (10 B/param), then clip (no grad read) + step (32 B/param)."""
    import torch

    import torchure_amd as ta
    from torchure_amd.optimizer.working import accumulate_grads_

    params, work, opt, n_params = build_state(config, chunk_elems, dev)
    g = torch.Generator(device=dev).manual_seed(77)
    micro = [w.grad for w in work]
    for p in params:
        p.grad = torch.randn(p.shape, device=dev, generator=g) * 3e-3
    stream = torch.cuda.current_stream(dev)

    def one(ev=None):
        for w, m in zip(work, micro):
            w.grad = m
        if ev is not None:
            ev[0].record(stream)
        accumulate_grads_(params, last=True)
        if ev is not None:
            ev[1].record(stream)
        ta.clip_grad_norm(params, None, 1.0)
        opt.step()
        if ev is not None:
            ev[2].record(stream)

    for _ in range(warmup):
        one()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        one(evs[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    acc_ms = statistics.median(e[0].elapsed_time(e[1]) for e in evs)
    step_ms = statistics.median(e[1].elapsed_time(e[2]) for e in evs)
    out = dict(
        config=config + "-fp32acc",
        n_params=n_params,
        ms_per_iteration=wall * 1e3 / steps,
        last_microstep_accumulate_norm_ms=round(acc_ms, 4),
        accumulate_GBps=round(10 * n_params / (acc_ms * 1e-3) / 1e9, 1),
        step_ms=round(step_ms, 4),
        step_bytes_per_param=32,
        step_GBps=round(32 * n_params / (step_ms * 1e-3) / 1e9, 1),
    )
    del params, work, opt, micro
    torch.cuda.empty_cache()
    return out


def run_torch_gpu_reference(config: str, steps: int, warmup: int, dev):
    """The reference's own GPU path on the same device, for comparison: fp32 grads
    (the reference trains with fp32 .grad), torch._foreach_norm + stack + vector_norm,
    clamp(max_norm / (total + 1e-6), max=1), torch._foreach_mul_
    (torchure/core/grad_helper.py:17-33), torch.optim.AdamW(fused=True) with the two
    groups of torchure/optimizer/builder.py:37-43, then the bf16 cast autocast performs
    (torchure/train/trainer.py:374). Same synthetic steady state as the main leg."""
    import torch

    from torchure_amd.workloads import shapes_for

    shapes = shapes_for(config)
    g = torch.Generator(device=dev).manual_seed(4321)
    params = [torch.nn.Parameter(torch.randn(s, device=dev, generator=g) * 0.02) for s in shapes]
    for p in params:
        p.grad = (torch.randn(p.shape, device=dev, generator=g) * 1e-3).to(torch.bfloat16).float()
    groups = [{"params": [p for p in params if p.dim() >= 2], "weight_decay": 0.1},
              {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0}]
    opt = torch.optim.AdamW(groups, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=True)
    for p in params:
        st = opt.state[p]
        st["step"] = torch.tensor(1000.0, dtype=torch.float32, device=dev)
        st["exp_avg"] = torch.randn(p.shape, device=dev, generator=g) * 1e-4
        st["exp_avg_sq"] = torch.randn(p.shape, device=dev, generator=g).abs_() * 1e-8
    bf16 = [torch.empty(p.shape, dtype=torch.bfloat16, device=dev) for p in params]
    grads = [p.grad for p in params]

    def one(cast=True):
        norms = torch._foreach_norm(grads, 2.0)
        total = torch.linalg.vector_norm(torch.stack(norms), 2.0)
        coef = torch.clamp(1.0 / (total + 1e-6), max=1.0)
        torch._foreach_mul_(grads, coef)
        opt.step()
        if cast:
            torch._foreach_copy_(bf16, params)

    def timed(cast):
        for _ in range(warmup):
            one(cast)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            one(cast)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    ms = timed(True)
    ms_nocast = timed(False)
    n = sum(p.numel() for p in params)
    del params, grads, opt, bf16
    torch.cuda.empty_cache()
    return dict(config=config, ms_per_step=round(ms, 4), n_params=n,
                GBps_on_30B_basis=round(STEP_BYTES_PER_PARAM * n / (ms * 1e-3) / 1e9, 1),
                path="torch-ROCm: fp32 grads, _foreach_norm clip + _foreach_mul_, "
                     "AdamW(fused=True), bf16 cast (46 B/param moved)",
                ms_per_step_without_bf16_cast=round(ms_nocast, 4))


def run_fused_ce(reps: int, dev, with_reference: bool = True, d: int = 1024):
    """Chunked fused linear + CE on the Qwen3-0.6B head: 8192 tokens (2 x 4096),
    hidden 1024, vocab 151936 (tied embedding), bf16 activations, fp32 weight,
    forward + backward (or another hidden size `d`: 2560 is the Qwen3-4B head). Roofline:
    the three GEMMs, 6 * N * D * V flops, bf16 MFMA."""
    import torch

    from torchure_amd.loss import fused_linear_cross_entropy

    n, v = 8192, 151936
    head_name = {1024: "qwen3-0.6b", 2560: "qwen3-4b", 4096: "qwen3-8b", 5120: "qwen3-14b"}.get(d, "D %d" % d)
    g = torch.Generator(device=dev).manual_seed(0)
    hidden = torch.randn(n, d, device=dev, generator=g).to(torch.bfloat16)
    weight = torch.randn(v, d, device=dev, generator=g) * 0.02
    labels = torch.randint(0, v, (n,), device=dev, generator=g)
    labels[::50] = -100
    flops = 6.0 * n * d * v

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps

    def ours(chunk="auto"):  # "auto": MI355X sizing, the whole 8192-token call in one chunk
        h = hidden.detach().requires_grad_(True)
        w = weight.detach().requires_grad_(True)
        fused_linear_cross_entropy(h, w, labels, -100, chunk).backward()

    out = {"workload": "%s lm_head: N 8192, D %d, V 151936, fwd+bwd, chunk_size='auto'" % (head_name, d),
           "flops": flops, "ms": round(timed(ours), 4)}
    out["TFLOPs"] = round(flops / (out["ms"] * 1e-3) / 1e12, 1)
    out["frac_of_bf16_mfma_peak"] = round(out["TFLOPs"] / 2500.0, 4)
    out["default_chunk1024_ms"] = round(timed(lambda: ours(1024)), 4)

    def evaluate():  # no input needs a gradient: the logits GEMM and the row losses only
        with torch.no_grad():
            fused_linear_cross_entropy(hidden, weight, labels, -100, "auto")

    out["loss_only_ms"] = round(timed(evaluate), 4)
    out["loss_only_TFLOPs"] = round(2.0 * n * d * v / (out["loss_only_ms"] * 1e-3) / 1e12, 1)

    hidden32 = hidden.float()

    def ours_fp32_hidden():  # the trainer's call: fp32 hidden states inside bf16 autocast
        h = hidden32.detach().requires_grad_(True)
        w = weight.detach().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = fused_linear_cross_entropy(h, w, labels, -100, 4096)
        loss.backward()

    out["fp32_hidden_autocast_chunk4096_ms"] = round(timed(ours_fp32_hidden), 4)

    # The same two calls on a head that carries a bf16 working copy kept by the optimizer
    # (attach_bf16_working_params): the op reads the copy instead of casting the fp32 master.
    import torchure_amd as ta

    head = torch.nn.Parameter(weight.detach().clone())
    ta.attach_bf16_working_params([head])

    def ours_fp32_hidden_copy():
        h = hidden32.detach().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = fused_linear_cross_entropy(h, head, labels, -100, 4096)
        torch.autograd.grad(loss, (h, head))  # no accumulation into head.grad, as in the leg above

    def evaluate_copy():
        with torch.no_grad():
            fused_linear_cross_entropy(hidden, head, labels, -100, "auto")

    out["working_copy_fp32_hidden_autocast_chunk4096_ms"] = round(timed(ours_fp32_hidden_copy), 4)
    out["working_copy_loss_only_ms"] = round(timed(evaluate_copy), 4)
    del head, hidden32
    if with_reference:
        # The reference composition (torchure/loss/fused_linear_ce.py:31-127) as the tests'
        # checker restates it, its chunk math compiled with torch.compile as the reference does:
        # a timed baseline beside this build, never the thing measured.
        from oracle.torch_composition import chunk_fwd_reference, fused_linear_ce_reference

        comp = torch.compile(chunk_fwd_reference, dynamic=False)

        def ref():
            fused_linear_ce_reference(hidden, weight, labels, -100, 1024, chunk_fn=comp)

        hidden32 = hidden.float()

        def ref_fp32_hidden():  # the trainer's call on the reference side (chunk 4096, autocast)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                fused_linear_ce_reference(hidden32, weight, labels, -100, 4096, chunk_fn=comp)

        try:
            out["reference_compiled_ms"] = round(timed(ref), 4)
            out["speedup_vs_reference_compiled"] = round(out["reference_compiled_ms"] / out["ms"], 3)
            out["speedup_vs_reference_compiled_both_chunk1024"] = round(
                out["reference_compiled_ms"] / out["default_chunk1024_ms"], 3)
            out["reference_compiled_fp32_hidden_autocast_chunk4096_ms"] = round(timed(ref_fp32_hidden), 4)
            out["speedup_fp32_hidden_autocast_chunk4096"] = round(
                out["reference_compiled_fp32_hidden_autocast_chunk4096_ms"] / out["fp32_hidden_autocast_chunk4096_ms"], 3)
        except Exception as e:  # torch.compile unavailable: report, do not fail the bench
            out["reference_compiled_error"] = repr(e)[:200]
        del hidden32
    del hidden, weight, labels
    torch.cuda.empty_cache()
    return out


def run_ce_gemm(shapes, reps: int, dev, vocab: int = 151936):
    """The fused CE's three products per chunk shape (rows x dim), each this build's MFMA GEMM
    against torch.matmul (hipBLASLt) on the same bf16 operands, timed over `reps` launches after
    one warm-up: logits = h @ W^T (fused_linear_ce.py:38, tm_ce_logits_bf16), grad_h =
    grad_logits @ W (:52, the split-K tm_ce_grad_h_bf16 with its fixed-order reduction) and
    grad_W = grad_logits^T @ h (:57, tm_ce_grad_w_bf16)."""
    import torch

    from torchure_amd import _native

    lib, stream = _native.lib(), _native.stream_handle(dev)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    out = {"vocab": vocab, "reps": reps, "shapes": {}}
    g = torch.Generator(device=dev).manual_seed(0)
    for dim in sorted({d for _, d in shapes}):
        w = (torch.randn(vocab, dim, device=dev, generator=g) * 0.05).to(torch.bfloat16)
        for rows in [r for r, d in shapes if d == dim]:
            a = torch.randn(rows, vocab, device=dev, generator=g).to(torch.bfloat16)
            o = torch.empty((rows, dim), dtype=torch.bfloat16, device=dev)
            nb = lib.tm_ce_grad_h_workspace_bytes(rows, vocab, dim)
            ws = torch.empty(nb, dtype=torch.uint8, device=dev)
            ms_s = timed(lambda: _native.check(lib.tm_ce_grad_h_bf16(o.data_ptr(), a.data_ptr(), w.data_ptr(), rows,
                                                                     vocab, dim, ws.data_ptr(), nb, stream),
                                               "tm_ce_grad_h_bf16"))
            ms_l = timed(lambda: torch.matmul(a, w, out=o))
            fl = 2.0 * rows * vocab * dim
            h = torch.randn(rows, dim, device=dev, generator=g).to(torch.bfloat16)
            logits = torch.empty((rows, vocab), dtype=torch.bfloat16, device=dev)
            ms_lg = timed(lambda: _native.check(lib.tm_ce_logits_bf16(logits.data_ptr(), h.data_ptr(), w.data_ptr(),
                                                                      rows, vocab, dim, stream), "tm_ce_logits_bf16"))
            ms_lg_l = timed(lambda: torch.matmul(h, w.t(), out=logits))
            gw = torch.empty((vocab, dim), dtype=torch.bfloat16, device=dev)
            ms_gw = timed(lambda: _native.check(lib.tm_ce_grad_w_bf16(gw.data_ptr(), a.data_ptr(), h.data_ptr(), rows,
                                                                      vocab, dim, stream), "tm_ce_grad_w_bf16"))
            ms_gw_l = timed(lambda: torch.matmul(a.t(), h, out=gw))
            out["shapes"]["%dx%d" % (rows, dim)] = {
                "splitk_ms": round(ms_s, 4), "splitk_TFLOPs": round(fl / ms_s / 1e9, 1),
                "hipblaslt_ms": round(ms_l, 4), "hipblaslt_TFLOPs": round(fl / ms_l / 1e9, 1),
                "splits": nb // (rows * dim * 4),
                "logits_ms": round(ms_lg, 4), "logits_TFLOPs": round(fl / ms_lg / 1e9, 1),
                "logits_hipblaslt_ms": round(ms_lg_l, 4), "logits_hipblaslt_TFLOPs": round(fl / ms_lg_l / 1e9, 1),
                "grad_w_ms": round(ms_gw, 4), "grad_w_TFLOPs": round(fl / ms_gw / 1e9, 1),
                "grad_w_hipblaslt_ms": round(ms_gw_l, 4), "grad_w_hipblaslt_TFLOPs": round(fl / ms_gw_l / 1e9, 1)}
            del a, o, ws, h, logits, gw
        del w
    return out


def _cpu_topology():
    """(logical CPUs this process may run on, physical cores among them or None)."""
    try:
        cpus = set(os.sched_getaffinity(0))
    except AttributeError:
        cpus = set(range(os.cpu_count() or 1))
    cores, cur = set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in list(f) + [""]:
                if line.strip():
                    k, _, v = line.partition(":")
                    cur[k.strip()] = v.strip()
                    continue
                if cur.get("processor", "").isdigit() and int(cur["processor"]) in cpus:
                    cores.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
    except OSError:
        pass
    return len(cpus), (len(cores) if cores and (None, None) not in cores else None)


def _cpu_one(config: str, steps: int, seconds: float, threads: int):
    """The reference composition on torch CPU over the whole parameter set of ``config``:
    fp32 masters and grads (bf16-valued), two param groups, steady state at step 1000.
    Values are drawn once into small pools and tiled into the tensors (the step's time does
    not depend on them), so a 4B set is set up in seconds. At least ``steps`` timed steps,
    more until ``seconds`` of CPU work has been timed; the median step is reported."""
    import torch

    from oracle.torch_composition import make_reference_optimizer, reference_step
    from torchure_amd.workloads import shapes_for

    g = torch.Generator().manual_seed(99)
    pools = {k: torch.randn(1 << 22, generator=g) * sc for k, sc in
             (("p", 0.02), ("g", 1e-3), ("m", 1e-4), ("v", 1e-8))}
    pools["g"] = pools["g"].to(torch.bfloat16).float()
    pools["v"].abs_()

    def filled(shape, key):
        t = torch.empty(shape)
        flat, src = t.view(-1), pools[key]
        k = flat.numel() // src.numel()
        if k:  # one multithreaded copy of the pool, tiled
            flat[: k * src.numel()].view(k, -1).copy_(src.expand(k, -1))
        rest = flat.numel() - k * src.numel()
        if rest:
            flat[k * src.numel():].copy_(src[:rest])
        return t

    shapes = shapes_for(config)
    params = [torch.nn.Parameter(filled(s, "p")) for s in shapes]
    for p in params:
        p.grad = filled(p.shape, "g")
    opt = make_reference_optimizer(params)
    for p in params:
        st = opt.state[p]
        st["step"] = torch.tensor(1000.0)
        st["exp_avg"] = filled(p.shape, "m")
        st["exp_avg_sq"] = filled(p.shape, "v")
    bf16 = [torch.empty(p.shape, dtype=torch.bfloat16) for p in params]
    n = sum(p.numel() for p in params)
    reference_step(params, opt, 1.0, bf16)  # warm-up
    times = []
    while len(times) < steps or (sum(times) < seconds and len(times) < 100):
        t0 = time.perf_counter()
        reference_step(params, opt, 1.0, bf16)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    del params, opt, bf16
    return dict(config=config, n_params=n, tensors=len(shapes), ms_per_step=round(med * 1e3, 1),
                GBps=round(n * STEP_BYTES_PER_PARAM / med / 1e9, 3), timed_steps=len(times),
                timed_s=round(sum(times), 1))


def run_cpu_baseline(configs: list[str], steps: int, seconds: float):
    """The reference's torch calls composed as its clip + optimizer step + bf16 cast
    (torchure/core/grad_helper.py:17-33, torchure/optimizer/builder.py:31-46,
    torchure/train/trainer.py:374; oracle/torch_composition.py), on torch CPU with one
    thread per logical CPU this process may use, over the whole parameter set of each
    config. The first config is the headline; the others are reported under ``configs``."""
    import torch

    logical, physical = _cpu_topology()
    torch.set_num_threads(logical)
    runs = [_cpu_one(c, steps, seconds, logical) for c in configs]
    head = runs[0]
    return dict(
        value=head["GBps"],
        unit="GB/s",
        cores=logical,
        kind="reference",
        kind_note="the reference's own torch calls (foreach-norm clip, torch.optim.AdamW(fused=True) "
                  "with its two groups, bf16 cast) composed in oracle/torch_composition.py and run "
                  "on torch CPU; no code of this build runs in it",
        ms_per_step=head["ms_per_step"],
        logical_cpus=logical,
        physical_cores=physical,
        host_ram_gib=_host_ram_gib(),
        sample=(f"{head['config']}: the whole parameter set ({head['tensors']} tensors, "
                f"{head['n_params']} params), median of {head['timed_steps']} steps "
                f"({head['timed_s']} s timed) after 1 warm-up, {head['ms_per_step']} ms/step; "
                f"GB/s on the same 30 B/param basis; {logical} threads on {logical} logical CPUs "
                f"({physical} physical cores), host RAM {_host_ram_gib()} GiB"),
        configs={r["config"]: r for r in runs[1:]},
    )


def _host_ram_gib() -> str:
    """Total host memory from /proc/meminfo, or '?' where it cannot be read."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal:"):
                    return f"{int(line.split()[1]) / 2 ** 20:.0f}"
    except OSError:
        pass
    return "?"


def load_traffic(config: str):
    path = os.path.join(ROOT, "profiles", f"adamw_update_{config}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def main():
    args = parse()
    if args.alloc_conf:  # read by torch's allocator when it starts, so set before any import
        os.environ["PYTORCH_CUDA_ALLOC_CONF"] = args.alloc_conf
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "optimizer step has no cross-GPU path here", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    import warnings

    with warnings.catch_warnings(record=True) as caught:  # the allocator reads its settings here
        warnings.simplefilter("always")
        torch.empty(1, device=dev)
    ignored = [str(w.message) for w in caught if "not supported" in str(w.message)]
    import torchure_amd

    torchure_amd._native.lib()
    if args.mode == "kernels":
        run_kernels_only(args.config, args.reps, args.chunk_elems, dev, args.states,
                         [x for x in args.state_layouts.split(",") if x])
        return
    if args.mode == "ce":  # fused linear CE only (for rocprofv3)
        print(json.dumps(run_fused_ce(args.reps, dev, with_reference=False, d=args.ce_dim)), flush=True)
        return
    if args.mode == "ce-gemm":
        shapes = [tuple(int(x) for x in sh.split("x")) for sh in args.gemm_shapes.split(",") if sh]
        print(json.dumps(run_ce_gemm(shapes, args.reps, dev)), flush=True)
        return

    main_res = run_gpu(args.config, args.steps, args.warmup, args.chunk_elems, dev)
    print(f"[bench] {args.config}: {main_res}", file=sys.stderr, flush=True)
    extra = {}
    for cfg in [c for c in args.also.split(",") if c and c != args.config]:
        if cfg.endswith("-again"):
            r = run_gpu(cfg[: -len("-again")], args.steps, args.warmup, args.chunk_elems, dev)
            r["GBps"] = round(r["n_params"] * STEP_BYTES_PER_PARAM / (r["ms_per_step"] * 1e-3) / 1e9, 1)
            r["frac_of_peak"] = round(r["GBps"] / PEAK_HBM_GBS, 4)
            r["update_GBps"] = round(r["n_params"] * UPDATE_BYTES_PER_PARAM / (r["update_ms_mean"] * 1e-3) / 1e9, 1)
            r["update_frac_of_peak"] = round(r["update_GBps"] / PEAK_HBM_GBS, 4)
            extra[cfg] = r
            print(f"[bench] {cfg}: {r}", file=sys.stderr, flush=True)
            continue
        if cfg.endswith("-dropin") or cfg.endswith("-ddpbuckets"):
            bucketed = cfg.endswith("-ddpbuckets")
            base_cfg = cfg.rsplit("-", 1)[0]
            r = run_gpu_dropin(base_cfg, args.steps, args.warmup, args.chunk_elems, dev, buckets=bucketed)
            extra[cfg] = r
            print(f"[bench] {cfg}: {r}", file=sys.stderr, flush=True)
            continue
        if cfg.endswith("-eager"):
            r = run_gpu_eager(cfg[: -len("-eager")], args.steps, args.warmup, args.chunk_elems, dev)
            extra[cfg] = r
            print(f"[bench] {cfg}: {r}", file=sys.stderr, flush=True)
            continue
        if cfg.endswith("-fp32acc"):
            r = run_gpu_fp32acc(cfg[: -len("-fp32acc")], args.steps, args.warmup, args.chunk_elems, dev)
            extra[cfg] = r
            print(f"[bench] {cfg}: {r}", file=sys.stderr, flush=True)
            continue
        r = run_gpu(cfg, args.steps, args.warmup, args.chunk_elems, dev)
        r["GBps"] = round(r["n_params"] * STEP_BYTES_PER_PARAM / (r["ms_per_step"] * 1e-3) / 1e9, 1)
        r["frac_of_peak"] = round(r["GBps"] / PEAK_HBM_GBS, 4)
        extra[cfg] = r
        print(f"[bench] {cfg}: {r}", file=sys.stderr, flush=True)

    if args.fused_ce:
        ce = run_fused_ce(5, dev, with_reference=bool(args.torch_reference))
        extra["fused_linear_ce_qwen3-0.6b"] = ce
        print(f"[bench] fused linear CE: {ce}", file=sys.stderr, flush=True)

    if args.torch_reference:
        ref = run_torch_gpu_reference(args.config, max(5, min(args.steps, 20)), 2, dev)
        ref["speedup_of_this_build"] = round(ref["ms_per_step"] / main_res["ms_per_step"], 3)
        dropin = extra.get(args.config + "-dropin")
        if dropin:
            # same fp32-grad inputs as the reference path, no bf16 working copies
            ref["speedup_of_dropin_fp32grads"] = round(ref["ms_per_step_without_bf16_cast"] /
                                                       dropin["ms_per_step"], 3)
        extra["torch_rocm_reference_" + args.config] = ref
        print(f"[bench] torch-ROCm reference: {ref}", file=sys.stderr, flush=True)

    n = main_res["n_params"]
    ms = main_res["ms_per_step"]
    value = n * STEP_BYTES_PER_PARAM / (ms * 1e-3) / 1e9
    upd_gbs = n * UPDATE_BYTES_PER_PARAM / (main_res["update_ms_mean"] * 1e-3) / 1e9
    cpu = None
    cpu_cfgs = [c for c in args.cpu_configs.split(",") if c]
    if cpu_cfgs:
        if cpu_cfgs[0] != args.config:
            cpu_cfgs = [args.config] + [c for c in cpu_cfgs if c != args.config]
        torch.cuda.empty_cache()
        cpu = run_cpu_baseline(cpu_cfgs, args.cpu_steps, args.cpu_seconds)
    line = {
        "metric": "optimizer step ms + achieved HBM GB/s (% of peak), Qwen3-0.6B & 4B shapes",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (fp64 intermediates), bf16 grads/params",
        "data": "synthetic (seeded steady-state optimizer inputs; no dataset)",
        "config": {"workload": f"{args.config} optimizer step: clip 1.0 + AdamW + bf16 refresh",
                   "params": n, "tensors": main_res["n_tensors"], "bytes_per_param": STEP_BYTES_PER_PARAM,
                   "grad_dtype": "bf16", "alloc_conf": args.alloc_conf or os.environ.get("PYTORCH_CUDA_ALLOC_CONF", ""),
                   "alloc_conf_ignored_by_torch": ignored[0] if ignored else None},
        "frac_of_peak": round(value / PEAK_HBM_GBS, 4),
        "params_per_s": round(n / (ms * 1e-3), 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "adamw_update_kernel",
            "achieved": round(upd_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(upd_gbs / PEAK_HBM_GBS, 4),
            "traffic": load_traffic(args.config),
            "launch_ms_mean": round(main_res["update_ms_mean"], 4),
            "norm_ms_mean": round(main_res["norm_ms_mean"], 4),
            "device_copy_GBps": main_res["copy_GBps"],
            "device_copy": "tm_stream_copy of 4 GiB, the best 1:1 read/write stream measured on this "
                           "device with this library's launch shapes",
            "frac_of_device_copy": round(upd_gbs / main_res["copy_GBps"], 4),
            "torch_copy_GBps": main_res["torch_copy_GBps"],
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
