"""AdamW for MI355X: torch.optim.AdamW's API and state layout, one fused gfx950 launch.

Drop-in for the optimizer torchure builds at torchure/optimizer/builder.py:46
(``torch.optim.AdamW(param_groups, lr=..., betas=..., fused=True)``):

- constructor: same positional/keyword parameters as torch.optim.AdamW
  (torch/optim/adamw.py:20-49, validation of torch/optim/adam.py:35-113);
  amsgrad, maximize, capturable, differentiable, tensor lr/betas and
  fused=False raise NotImplementedError (RuntimeError for fused+foreach, as torch);
- ``param_groups`` carry exactly torch AdamW's keys (adam.py:91-103, with
  decoupled_weight_decay=True), so schedulers that read/write ``lr`` and
  ``initial_lr`` work unchanged (torch/optim/lr_scheduler.py:135-145,284-297);
- per-param state is ``{'step': fp32 0-d tensor on the param's device,
  'exp_avg', 'exp_avg_sq'}`` created lazily on the first step that sees a grad
  (adam.py:139-212), so ``state_dict()``/``load_state_dict()`` round-trip with
  torch.optim.AdamW checkpoints in both directions
  (torch/optim/optimizer.py:677-767,877-1014; torchure/checkpoint/checkpointer.py:43-60);
- params whose grad is None are skipped and their step does not advance
  (adam.py:150-153); all-zero grads still update.

One ``step()`` is one native call (``tm_adamw_step``) per device covering
every group and tensor: a tiny prep kernel (step += 1, fp64 bias corrections)
and one update kernel that reads grad/master/m/v once and writes
master/m/v and, when a bf16 working copy is attached, RNE(master) once.

Mixed precision: masters are the fp32 ``nn.Parameter``s, as in the reference
(torchure/train/trainer.py:246-262). A master may carry a bf16 working copy
(``torchure_amd.optimizer.working``); when its own ``.grad`` is None the bf16
grad of the working copy is consumed, and the working copy is refreshed with
RNE(master) after the update.
"""

from __future__ import annotations

import numpy as np
import torch
import weakref

from torchure_amd import _native
from torchure_amd.core import tables

class _Owner:
    """``p._tm_owner``: a weak reference to the AdamW that holds ``p``; calling it gives that
    optimizer, or None once it is gone. Pickling and copying give an empty mark (a saved or
    copied param belongs to no optimizer), so ``torch.save(model)`` and ``copy.deepcopy`` work
    as with torch's own optimizers, which leave params untouched."""

    __slots__ = ("ref",)

    def __init__(self, opt=None):
        self.ref = weakref.ref(opt) if opt is not None else None

    def __call__(self):
        return self.ref() if self.ref is not None else None

    def __reduce__(self):
        return (_Owner, ())

    def __copy__(self):
        return _Owner()

    def __deepcopy__(self, memo):
        return _Owner()


# The owner mark of a param held by more than one AdamW: it reads as no owner, so a clip over
# it scales the grads in place (every optimizer then sees them scaled, as in the reference)
# instead of deferring the scale into one of them.
_SHARED = _Owner()


def owner_of(p: torch.Tensor):
    """The torchure_amd AdamW that owns ``p`` (a weak reference set by add_param_group), or None
    (no owner, or several)."""
    ref = getattr(p, "_tm_owner", None)
    return ref() if ref is not None else None


def owners_of(params) -> set:
    """Set of owners (AdamW objects, or None for unowned params) of ``params``."""
    out = set()
    for p in params:
        ref = getattr(p, "_tm_owner", None)
        out.add(ref() if ref is not None else None)
    return out


def materialize_pending_for(params, owners=None) -> None:
    """Apply any deferred clip pending on the optimizers that own ``params``."""
    for opt in owners if owners is not None else owners_of(params):
        if opt is not None and opt._pending is not None:
            opt.materialize_clip()


class AdamW(torch.optim.Optimizer):
    def __init__(
        self,
        params,
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
        amsgrad: bool = False,
        *,
        maximize: bool = False,
        foreach: bool | None = None,
        capturable: bool = False,
        differentiable: bool = False,
        fused: bool | None = None,
        chunk_elems: int = tables.DEFAULT_CHUNK_ELEMS,
        defer_clip: bool = True,
    ) -> None:
        if isinstance(lr, torch.Tensor) or any(isinstance(b, torch.Tensor) for b in betas):
            raise NotImplementedError("torchure_amd.AdamW: tensor lr/betas are not supported")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if amsgrad:
            raise NotImplementedError("torchure_amd.AdamW: amsgrad is not supported")
        if maximize:
            raise NotImplementedError("torchure_amd.AdamW: maximize is not supported")
        if capturable:
            raise NotImplementedError("torchure_amd.AdamW: capturable is not supported")
        if differentiable:
            raise NotImplementedError("torchure_amd.AdamW: differentiable is not supported")
        if fused is False:
            raise NotImplementedError("torchure_amd.AdamW is always fused; fused=False is not supported")
        if foreach:
            raise RuntimeError("`fused` and `foreach` cannot be `True` together.")
        defaults = {
            "lr": lr,
            "betas": (float(betas[0]), float(betas[1])),
            "eps": eps,
            "weight_decay": weight_decay,
            "amsgrad": False,
            "maximize": False,
            "foreach": foreach,
            "capturable": False,
            "differentiable": False,
            "fused": True,
            "decoupled_weight_decay": True,
        }
        self.chunk_elems = tables.check_chunk_elems(chunk_elems)
        self.defer_clip = bool(defer_clip)
        self._pending = None  # (coef device tensor, _ClipRecord)
        self._uploader = tables.TableUploader()
        self._verified: dict = {}  # id(param) -> _ParamEntry
        self._plan = None  # _Plan of the last full step, reused while nothing changes
        super().__init__(params, defaults)

    def add_param_group(self, param_group: dict) -> None:
        # checked first, so a refused group leaves the optimizer as it was
        if len(self.param_groups) >= _native.TM_MAX_GROUPS:
            raise ValueError(f"torchure_amd.AdamW: at most {_native.TM_MAX_GROUPS} param groups")
        super().add_param_group(param_group)
        self._mark_owned(self.param_groups[-1]["params"])
        self._plan = None

    def _mark_owned(self, params) -> None:
        own = _Owner(self)
        for p in params:
            cur = getattr(p, "_tm_owner", None)
            if cur is _SHARED:
                continue
            prev = cur() if cur is not None else None
            p._tm_owner = own if prev is None or prev is self else _SHARED

    def __getstate__(self):
        """torch's pickled state (defaults, state, param_groups) plus this optimizer's settings."""
        state = super().__getstate__()
        state["chunk_elems"] = self.chunk_elems
        state["defer_clip"] = self.defer_clip
        return state

    def __setstate__(self, state):
        super().__setstate__(state)
        for group in self.param_groups:
            group["decoupled_weight_decay"] = True
            self._mark_owned(group["params"])
        self.__dict__.setdefault("chunk_elems", tables.DEFAULT_CHUNK_ELEMS)
        self.__dict__.setdefault("defer_clip", True)
        self.__dict__.setdefault("_pending", None)
        self.__dict__.setdefault("_uploader", tables.TableUploader())
        self.__dict__.setdefault("_verified", {})
        self.__dict__.setdefault("_plan", None)

    # ------------------------------------------------------------ deferred clip

    def _set_pending_clip(self, coef: torch.Tensor, params, grads) -> None:
        """Defer ``grads *= coef`` into the next step. Each grad is recorded with its
        autograd version: the reference scales at clip time, so a grad modified in
        place before the step cannot be reproduced by scaling later (the step raises),
        while a grad replaced by a new tensor simply steps unscaled, as it would there."""
        grads = list(grads)
        self._pending = (coef, _ClipRecord(list(params), grads, _native.host().versions(grads)))

    @staticmethod
    def _modified_error() -> RuntimeError:
        return RuntimeError(
            "torchure_amd.AdamW: a grad was modified in place after clip_grad_norm deferred its "
            "scaling into this optimizer; call optimizer.materialize_clip() before changing grads "
            "between clip_grad_norm and step(), or build the optimizer with defer_clip=False")

    def materialize_clip(self) -> None:
        """Apply a pending clip coefficient to the grads it measured, in place, and drop it."""
        if self._pending is None:
            return
        coef, rec = self._pending
        from torchure_amd.core.grad_helper import scale_grads_

        if not np.array_equal(_native.host().versions(rec.grads), rec.versions):
            raise self._modified_error()  # the clip stays pending, as after a refused step()
        self._pending = None
        scale_grads_(rec.grads, coef)

    # ------------------------------------------------------------ step

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        pending = self._pending
        coef, clip_ids = pending if pending is not None else (None, ())
        # a refused step (a grad changed in place since the clip) keeps the clip pending, so
        # a second step() refuses too instead of stepping on unscaled grads; zero_grad() drops it
        launches = self.plan_step(coef, clip_ids)
        self._pending = None
        for launch in launches:
            launch()
        return loss

    @torch.no_grad()
    def plan_step(self, coef: torch.Tensor | None = None, clip_ids=()) -> list["StepLaunch"]:
        """Collect the params with grads (creating their state lazily) and return
        the native launches of one step without running them. ``step()`` runs
        them once; calling a launch again applies one more step to the same
        tensors and grads (bench.py uses this to time the kernels back to back).

        ``clip_ids`` names the params whose grads are multiplied by ``coef``: a set of
        ids, or the record of a deferred clip, which is checked (same grad objects, same
        autograd versions)."""
        fast = self._plan_fast(coef, clip_ids)
        if fast is not None:
            return fast
        self._plan = None
        self._init_states_pooled()
        order = []  # (param, entry) of every param with a grad, in table order
        rec = clip_ids if isinstance(clip_ids, _ClipRecord) else None
        if rec is not None:
            clip_ids = rec.index
            rec_grads = rec.grads
            vsum = 0  # versions now, of the recorded grads that are still the params' grads
            matched = []
        per_dev: dict = {}
        hyper = []
        state_map = self.state
        verified = self._verified
        clip_flag = _native.TM_FLAG_CLIP
        bf16, f32 = torch.bfloat16, torch.float32
        for gi, group in enumerate(self.param_groups):
            lr = group["lr"]
            if isinstance(lr, torch.Tensor):
                raise NotImplementedError("torchure_amd.AdamW: tensor lr is not supported")
            beta1, beta2 = group["betas"]
            for key in ("amsgrad", "maximize", "capturable", "differentiable"):
                if group.get(key):
                    raise NotImplementedError(f"torchure_amd.AdamW: {key}=True is not supported")
            hyper.append((float(lr), float(beta1), float(beta2), float(group["weight_decay"]), float(group["eps"])))
            for p in group["params"]:
                g = p.grad
                work = getattr(p, "_tm_working", None)
                if g is None:
                    if work is None:
                        continue
                    g = work.grad
                    if g is None:
                        continue
                state = state_map[p]
                ent = verified.get(id(p))
                # same objects and same storage: a `.data =` swap on any of them (which
                # frees the old storage) must not leave a stale pointer in the table
                if (ent is None or ent.param is not p or ent.work is not work
                        or state.get("step") is not ent.step or state.get("exp_avg") is not ent.m
                        or state.get("exp_avg_sq") is not ent.v or p.data_ptr() != ent.p_ptr
                        or ent.m.data_ptr() != ent.m_ptr or ent.v.data_ptr() != ent.v_ptr
                        or ent.step.data_ptr() != ent.s_ptr
                        or (work is not None and work.data_ptr() != ent.w_ptr)):
                    ent = self._verify_param(p, state, work)
                    verified[id(p)] = ent
                gdt = g.dtype
                if gdt is bf16:
                    flags = _native.TM_GRAD_BF16
                elif gdt is f32:
                    flags = _native.TM_GRAD_F32
                else:
                    flags = tables.grad_flags(g, "torchure_amd.AdamW")  # raises
                if (g.is_sparse or not g.is_cuda or g.get_device() != ent.dev_index
                        or g.numel() != ent.numel or not g.is_contiguous()):
                    self._check_param(p, g, work)  # raises with a precise message
                if rec is None:
                    if id(p) in clip_ids:
                        flags |= clip_flag
                else:
                    k = clip_ids.get(id(p))
                    # a grad replaced since the clip steps unscaled, as in the reference
                    if k is not None and rec_grads[k] is g:
                        flags |= clip_flag
                        vsum += g._version
                        matched.append(k)
                if work is not None and getattr(work, "_tm_master_version", None) != p._version:
                    raise RuntimeError(
                        "torchure_amd.AdamW: a fp32 master was modified in place since its "
                        "bf16 working copy was last written, so the forward ran on stale "
                        "weights; call torchure_amd.refresh_bf16_working_params(params) "
                        "after changing masters (e.g. after model.load_state_dict)")
                bucket = per_dev.get(ent.device)
                if bucket is None:
                    bucket = per_dev[ent.device] = ([], [], [])
                bucket[0].append((ent.p_ptr, ent.m_ptr, ent.v_ptr, g.data_ptr(), ent.w_ptr, ent.s_ptr,
                                  ent.numel, gi, flags))
                bucket[1].extend(ent.written)
                if work is not None:
                    bucket[2].append(ent)
                order.append((p, ent))

        if rec is not None:
            vers = rec.versions
            want = rec.total if len(matched) == len(vers) else sum(vers[k] for k in matched)
            if vsum != want:  # versions only grow: any in-place change since the clip shows here
                raise self._modified_error()
        if not per_dev:
            return []
        launches = self._plan_launches(per_dev, hyper, coef)
        if len(launches) == 1:
            self._plan = _Plan(self, order, launches[0])
        return launches

    def _plan_fast(self, coef, clip_ids):
        """The steady-state step: the same params have grads from the same sources, and
        every cached pointer, state object and working-copy version still holds. Then only
        the grad pointers (and the clip flags) of the cached table change. Returns None
        whenever anything differs; the full per-param path then rebuilds the plan and
        reports any error precisely."""
        plan = self._plan
        if plan is None or plan.chunk_elems != self.chunk_elems:
            return None
        groups = self.param_groups
        if len(groups) != len(plan.groups):
            return None
        host = _native.host()
        for group, (g0, plist, snap) in zip(groups, plan.groups):
            if group is not g0 or group["params"] is not plist or not host.same(plist, snap):
                return None
        hyper = []
        for group in groups:
            lr = group["lr"]
            if isinstance(lr, torch.Tensor) or any(group.get(k) for k in _UNSUPPORTED):
                return None
            b1, b2 = group["betas"]
            hyper.append((float(lr), float(b1), float(b2), float(group["weight_decay"]), float(group["eps"])))
        if not host.attrs_same(plan.all_params, "_tm_working", plan.all_works):
            return None
        gs, src = host.grads(plan.all_params, plan.all_works)
        if src != plan.src:
            return None
        gl = [g for g in gs if g is not None]
        if not host.dense_contiguous(gl) or not np.array_equal(host.ptrs(plan.statics), plan.static_ptrs):
            return None
        if not host.states_same(self.state, plan.params, plan.states, plan.ms, plan.vs, plan.ss):
            return None
        if plan.wparams and not host.stamped(plan.wparams, plan.wworks):
            return None
        flags = plan.flags
        if coef is not None and clip_ids:
            if not isinstance(clip_ids, _ClipRecord) or len(clip_ids.grads) != len(gl):
                return None
            rec = clip_ids
            if plan.clip_holders is None or not host.same(rec.holders, plan.clip_holders):
                perm = [rec.index.get(id(p)) for p in plan.params]
                if None in perm:
                    return None
                plan.clip_holders, plan.clip_perm = rec.holders, perm
            rg = rec.grads
            if not host.same([rg[k] for k in plan.clip_perm], gl):
                return None
            if host.version_sum(gl) != rec.total:
                raise self._modified_error()
            flags = flags | _native.TM_FLAG_CLIP
        device = plan.device
        if coef is not None and coef.device != device:
            return None
        rows = plan.rows.copy()
        rows["grad"] = host.ptrs(gl)
        rows["flags"] = flags
        tables.make_ready(plan.chunks, device)
        return [StepLaunch(device, self._uploader(rows, device), plan.n, plan.chunks, plan.n_chunks,
                           self.chunk_elems, _native.hyper_array(hyper), len(hyper), coef,
                           plan.written, (plan.wparams, plan.wworks))]

    @torch.no_grad()
    def init_state(self) -> None:
        """Create the lazy state of every param that has a grad and no state yet, as the next
        step() would (step 0, zero moments, in the pooled layout), without stepping. Lets a
        caller place or fill the state (a resume, a benchmark) before the first step."""
        self._init_states_pooled()

    def _init_states_pooled(self) -> None:
        """Lazy state of every param that has a grad and no state yet (torch creates it at
        the first step that sees a grad, adam.py:139-212), created together: per device, one
        fp32 buffer per role (exp_avg, exp_avg_sq) holds all of them, and each param's moment
        is a view of it (``pooled_layout``), so the update streams two large arrays laid out
        the same way instead of hundreds of allocations wherever the caching allocator put
        them. ``step`` stays a 0-d fp32 tensor per param, as torch keeps it."""
        fresh = []
        state_map = self.state
        for group in self.param_groups:
            for p in group["params"]:
                if state_map.get(p):
                    continue
                work = getattr(p, "_tm_working", None)
                if p.grad is None and (work is None or work.grad is None):
                    continue
                if p.is_cuda and p.dtype == torch.float32 and p.is_contiguous() and not p.is_sparse:
                    fresh.append(p)  # anything else is refused, precisely, by _verify_param
        if fresh:
            with torch.no_grad():
                for p, m, v in pooled_moments(fresh, zero=True):
                    state_map[p] = {"step": torch.zeros((), dtype=torch.float32, device=p.device),
                                    "exp_avg": m, "exp_avg_sq": v}

    def _verify_param(self, p: torch.Tensor, state: dict, work) -> "_ParamEntry":
        """Full checks of a param, its working copy and its state (created lazily,
        moved to fp32 on the param's device when loaded from elsewhere); cached
        until any of those objects changes."""
        who = "torchure_amd.AdamW"
        tables.require_device_tensor(p, who, "param")
        if p.dtype != torch.float32:
            raise RuntimeError(f"{who}: params (fp32 masters) must be float32, got {p.dtype}")
        if work is not None:
            tables.require_device_tensor(work, who, "bf16 working copy")
            if work.dtype != torch.bfloat16 or work.numel() != p.numel() or work.device != p.device:
                raise RuntimeError(f"{who}: working copy must be bf16 of the param's size and device")
        if len(state) == 0:
            state["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
            state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
            state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
        else:
            st = state["step"]
            if st.device != p.device or st.dtype != torch.float32:
                state["step"] = st.to(dtype=torch.float32, device=p.device)
            for k in ("exp_avg", "exp_avg_sq"):
                t = state[k]
                if t.numel() != p.numel():
                    raise RuntimeError(f"{who}: state['{k}'] has {t.numel()} elements, param {p.numel()}")
                if t.device != p.device or t.dtype != torch.float32 or not t.is_contiguous():
                    state[k] = t.to(dtype=torch.float32, device=p.device).contiguous()
        return _ParamEntry(p, work, state["step"], state["exp_avg"], state["exp_avg_sq"])

    def load_state_dict(self, state_dict) -> None:
        """torch's loader (torch/optim/optimizer.py:877-1014), then the groups say what runs.
        torch copies the saved groups' flags over the live ones, so a checkpoint of a
        non-fused AdamW would leave ``fused=None`` here; this optimizer always runs the fused
        recipe, and its groups say so again (``state_dict()`` then reports what ran). Step
        counters that torch's policy leaves on the CPU for such checkpoints are moved to the
        param's device, as fp32, by the first step."""
        self._verified.clear()
        self._plan = None
        super().load_state_dict(state_dict)
        for group in self.param_groups:
            group["fused"] = True
            group["foreach"] = None
        self._repack_states()

    def _repack_states(self) -> None:
        """Moments loaded from a checkpoint (separate tensors, or views of a loaded storage)
        are copied into this optimizer's pooled layout, as if created by its first step."""
        held = []
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if not st or not (p.is_cuda and p.dtype == torch.float32 and p.is_contiguous()):
                    continue
                m, v = st.get("exp_avg"), st.get("exp_avg_sq")
                if (isinstance(m, torch.Tensor) and isinstance(v, torch.Tensor) and m.numel() == p.numel()
                        and v.numel() == p.numel() and m.dtype == v.dtype == torch.float32
                        and m.device == v.device == p.device):
                    held.append((p, st, m, v))
        if not held:
            return
        with torch.no_grad():
            for (p, st, m, v), (_, pm, pv) in zip(held, pooled_moments([h[0] for h in held], zero=False)):
                pm.copy_(m.reshape(pm.shape))
                pv.copy_(v.reshape(pv.shape))
                st["exp_avg"], st["exp_avg_sq"] = pm, pv

    def _plan_launches(self, per_dev, hyper, coef) -> list["StepLaunch"]:
        groups_c = _native.hyper_array(hyper)
        out = []
        for device, (recs, written, pairs) in per_dev.items():
            n = len(recs)
            rows = np.array(recs, dtype=_native.TENSOR_DTYPE)
            if coef is not None and coef.device != device:
                raise RuntimeError("torchure_amd.AdamW: clip coefficient on another device")
            chunks, n_chunks = tables.CHUNKS.get(rows["numel"], self.chunk_elems, device)
            launch = StepLaunch(device, self._uploader(rows, device), n, chunks, n_chunks,
                                self.chunk_elems, groups_c, len(hyper), coef, written,
                                ([e.param for e in pairs], [e.work for e in pairs]))
            launch.host_rows = rows.tobytes()
            out.append(launch)
        return out

    @staticmethod
    def _check_param(p: torch.Tensor, g: torch.Tensor, work) -> None:
        who = "torchure_amd.AdamW"
        tables.require_device_tensor(p, who, "param")
        if p.dtype != torch.float32:
            raise RuntimeError(f"{who}: params (fp32 masters) must be float32, got {p.dtype}")
        if g.is_sparse:
            raise RuntimeError("Adam does not support sparse gradients, please consider SparseAdam instead")
        tables.require_device_tensor(g, who, "grad")
        if g.device != p.device or g.numel() != p.numel():
            raise RuntimeError(f"{who}: grad of shape {tuple(g.shape)} on {g.device} does not match "
                               f"param {tuple(p.shape)} on {p.device}")
        if work is not None:
            tables.require_device_tensor(work, who, "bf16 working copy")
            if work.dtype != torch.bfloat16 or work.numel() != p.numel() or work.device != p.device:
                raise RuntimeError(f"{who}: working copy must be bf16 of the param's size and device")

    def zero_grad(self, set_to_none: bool = True) -> None:
        self._pending = None
        super().zero_grad(set_to_none=set_to_none)
        for group in self.param_groups:
            for p in group["params"]:
                w = getattr(p, "_tm_working", None)
                if w is not None and w.grad is not None:
                    if set_to_none:
                        w.grad = None
                    else:
                        w.grad.zero_()


class _ParamEntry:
    """Verified per-param record: the objects it was built from and their pointers."""

    __slots__ = ("param", "work", "step", "m", "v", "p_ptr", "m_ptr", "v_ptr", "s_ptr", "w_ptr",
                 "numel", "device", "dev_index", "written")

    def __init__(self, p, work, step, m, v):
        self.param, self.work, self.step, self.m, self.v = p, work, step, m, v
        # tensors the step writes through raw pointers; their autograd version counters
        # are bumped after each launch, as an in-place torch op would do
        self.written = (p, m, v, step) if work is None else (p, m, v, step, work)
        self.p_ptr = p.data_ptr()
        self.m_ptr = m.data_ptr()
        self.v_ptr = v.data_ptr()
        self.s_ptr = step.data_ptr()
        self.w_ptr = work.data_ptr() if work is not None else 0
        self.numel = p.numel()
        self.device = p.device
        self.dev_index = p.get_device()


class _ClipRecord:
    """A deferred clip: the params whose grads it measured, those grad objects and their
    autograd versions at clip time (``index`` maps id(param) to its position)."""

    __slots__ = ("holders", "grads", "versions", "total", "_index")

    def __init__(self, holders: list, grads: list, versions):
        self.holders, self.grads, self.versions = holders, grads, versions
        self.total = int(np.asarray(versions, dtype=np.int64).sum())
        self._index = None

    @property
    def index(self) -> dict:
        if self._index is None:
            self._index = dict(zip(map(id, self.holders), range(len(self.holders))))
        return self._index


_UNSUPPORTED = ("amsgrad", "maximize", "capturable", "differentiable")


class _Plan:
    """The table of the last full step and what it was built from, for the fast path."""

    __slots__ = ("groups", "all_params", "all_works", "src", "params", "statics", "static_ptrs",
                 "states", "ms", "vs", "ss", "wparams", "wworks", "rows", "flags", "n", "device",
                 "chunks", "n_chunks", "chunk_elems", "written", "clip_holders", "clip_perm")

    def __init__(self, opt: "AdamW", order: list, launch: "StepLaunch"):
        host = _native.host()
        # each group, its params list and a snapshot of that list's contents
        self.groups = [(g, g["params"], list(g["params"])) for g in opt.param_groups]
        self.all_params = [p for g in opt.param_groups for p in g["params"]]
        self.all_works = [getattr(p, "_tm_working", None) for p in self.all_params]
        self.src = host.grads(self.all_params, self.all_works)[1]
        self.params = [p for p, _ in order]
        ents = [e for _, e in order]
        self.statics = [t for e in ents for t in (e.param, e.m, e.v, e.step, e.work)]
        self.static_ptrs = host.ptrs(self.statics)
        self.states = [opt.state[p] for p in self.params]
        self.ms = [e.m for e in ents]
        self.vs = [e.v for e in ents]
        self.ss = [e.step for e in ents]
        self.wparams, self.wworks = launch.pair_params, launch.pair_works
        self.n = launch.n
        self.device = launch.device
        self.chunks, self.n_chunks, self.chunk_elems = launch.chunks, launch.n_chunks, launch.chunk_elems
        self.written = launch.written
        self.rows = np.frombuffer(launch.host_rows, dtype=_native.TENSOR_DTYPE).copy()
        self.flags = self.rows["flags"] & ~np.uint32(_native.TM_FLAG_CLIP)
        self.clip_holders = None
        self.clip_perm = None


class StepLaunch:
    """One ``tm_adamw_step`` call with its device tables kept alive.

    Calling it enqueues the prep + update kernels on the device's current
    stream. Calling it again re-applies one more AdamW step to the same
    tensors with the same grads (used to time the kernels back to back).
    A call on a stream other than the one it was planned on first waits for
    that stream, where its table was uploaded.
    """

    def __init__(self, device, d_rows, n, chunks, n_chunks, chunk_elems, groups_c, n_groups, coef,
                 written=(), pairs=((), ())):
        self.written = written if isinstance(written, list) else list(written)
        # the masters with a working copy, and those copies
        self.pair_params, self.pair_works = (x if isinstance(x, list) else list(x) for x in pairs)
        self.host_rows = None  # the uploaded table's bytes, when the caller keeps them
        self.device = device
        self.d_rows = d_rows
        self.n = n
        self.chunks = chunks
        self.n_chunks = n_chunks
        self.chunk_elems = chunk_elems
        self.groups_c = groups_c
        self.n_groups = n_groups
        self.coef = coef
        self.ws = torch.empty(_native.workspace_bytes(n), dtype=torch.uint8, device=device)
        self.home = torch.cuda.current_stream(device)  # where the table was uploaded

    def __call__(self) -> None:
        tables.follow_home_stream(self.home, self.device, (self.d_rows, self.chunks, self.ws))
        rc = _native.lib().tm_adamw_step(
            self.d_rows.data_ptr(),
            self.n,
            self.chunks.data_ptr(),
            self.n_chunks,
            self.chunk_elems,
            self.groups_c,
            self.n_groups,
            self.coef.data_ptr() if self.coef is not None else None,
            self.ws.data_ptr(),
            _native.stream_handle(self.device),
        )
        _native.check(rc, "tm_adamw_step")
        if self.written:
            _native.host().bump(self.written)
        if self.pair_params:  # the copies now hold RNE(master) as of the versions after the bump
            _native.host().stamp(self.pair_params, self.pair_works)


POOL_ALIGN_ELEMS = 256  # 1 KiB of fp32: the update's slices start on these boundaries


def pooled_layout(numels, phases=None) -> tuple[list[int], int]:
    """Offsets (elements) of tensors of ``numels`` elements in one fp32 pool that starts on a
    1 KiB boundary, and the pool's length.

    ``phases[i]`` is the position (elements, a multiple of 4 below 256) past a 1 KiB boundary
    at which tensor i must start, or None for any 16-byte aligned start. The optimizer passes
    each master's own phase, so that a param's master, exp_avg and exp_avg_sq all sit at the
    same distance from a 1 KiB boundary and the update's slices start on one in all three.
    Tensors are placed greedily: the next one is a tensor whose phase is the current
    position's, lengths that are multiples of 256 first (they keep the position's phase), in
    the given order; when none is left for the current phase, the position moves to the
    nearest phase ahead that still has tensors. Tensors with no phase come last, each rounded
    up to 4 elements. With ``phases`` None every tensor whose length is a multiple of 256 gets
    phase 0 and the others none. Qwen3 sets need no padding when their masters sit on 1 KiB
    boundaries (the 128-wide q/k norms, shorter than a slice, take no phase)."""
    n_t = len(numels)
    if phases is None:
        phases = [0 if n % POOL_ALIGN_ELEMS == 0 else None for n in numels]
    offs = [0] * n_t
    buckets: dict = {}
    free = []
    for i, (n, ph) in enumerate(zip(numels, phases)):
        if ph is None:
            free.append(i)
        else:
            buckets.setdefault(int(ph) % POOL_ALIGN_ELEMS, ([], []))[0 if n % POOL_ALIGN_ELEMS == 0 else 1].append(i)
    for whole, rest in buckets.values():  # popped from the end: keep the given order
        whole.reverse()
        rest.reverse()
    pos, left = 0, n_t - len(free)
    while left:
        b = buckets.get(pos % POOL_ALIGN_ELEMS)
        if b is not None and (b[0] or b[1]):
            i = b[0].pop() if b[0] else b[1].pop()
            offs[i] = pos
            pos += (numels[i] + 3) // 4 * 4
            left -= 1
            continue
        cur = pos % POOL_ALIGN_ELEMS
        pos += min((ph - cur) % POOL_ALIGN_ELEMS for ph, bb in buckets.items() if bb[0] or bb[1])
    for i in free:
        offs[i] = pos
        pos += (numels[i] + 3) // 4 * 4
    return offs, pos


def master_phase(p: torch.Tensor):
    """Elements from the 1 KiB boundary at or before ``p``'s first element, for a 16-byte
    aligned fp32 tensor (the update's grid phase of that array); None otherwise."""
    ptr = p.data_ptr()
    return (ptr // 4) % POOL_ALIGN_ELEMS if ptr % 16 == 0 else None


def _aligned_pool(total: int, device, zero: bool) -> torch.Tensor:
    """An fp32 buffer of ``total`` elements starting on a 1 KiB boundary. Large blocks from the
    caching allocator already do; a block that does not is allocated again with 1 KiB more and
    viewed from its first boundary."""
    make = torch.zeros if zero else torch.empty
    buf = make(max(total, 1), dtype=torch.float32, device=device)
    if buf.data_ptr() % (4 * POOL_ALIGN_ELEMS) == 0:
        return buf
    buf = make(total + POOL_ALIGN_ELEMS, dtype=torch.float32, device=device)
    skip = (-buf.data_ptr() // 4) % POOL_ALIGN_ELEMS
    return buf[skip: skip + total]


def pooled_moments(params, zero: bool = True):
    """(param, exp_avg view, exp_avg_sq view) for ``params``: per device, one pool per role
    with ``pooled_layout`` at the params' own phases, the same layout in both pools, so each
    param's master and two moments sit at the same distance from a 1 KiB boundary."""
    per_dev: dict = {}
    for p in params:
        per_dev.setdefault(p.device, []).append(p)
    out = {}
    for device, ps in per_dev.items():
        # a tensor shorter than one 256-element slice is covered by one wave wherever it sits
        phases = [master_phase(p) if p.numel() >= POOL_ALIGN_ELEMS else None for p in ps]
        offs, total = pooled_layout([p.numel() for p in ps], phases)
        pm, pv = _aligned_pool(total, device, zero), _aligned_pool(total, device, zero)
        for p, o in zip(ps, offs):
            n = p.numel()
            out[id(p)] = (pm[o: o + n].view(p.shape), pv[o: o + n].view(p.shape))
    return [(p, *out[id(p)]) for p in params]


def step_bytes_per_param(grad_bytes: int, with_norm: bool = True, with_bf16_out: bool = True) -> int:
    """Algorithmic HBM bytes per parameter of one step (norm pass + update)."""
    upd = grad_bytes + 3 * 4 + 3 * 4 + (2 if with_bf16_out else 0)
    return upd + (grad_bytes if with_norm else 0)


__all__ = ["AdamW", "owner_of", "owners_of", "materialize_pending_for", "step_bytes_per_param",
           "pooled_layout", "pooled_moments", "master_phase"]
