"""Host-side API of the drop-in (no GPU): constructor, groups, schedule, state layout, errors."""

from __future__ import annotations

import os

import pytest
import torch

import torchure_amd as ta
from oracle import oracle
from torchure_amd.optimizer import AdamW, build_optimizer, build_scheduler, wsd_scale


def _model():
    return torch.nn.Sequential(torch.nn.Linear(8, 4), torch.nn.LayerNorm(4), torch.nn.Linear(4, 2, bias=False))


def test_constructor_rejects_unsupported():
    p = [torch.nn.Parameter(torch.zeros(3))]
    for kw in ({"amsgrad": True}, {"maximize": True}, {"capturable": True}, {"differentiable": True},
               {"fused": False}):
        with pytest.raises(NotImplementedError):
            AdamW(p, **kw)
    with pytest.raises(RuntimeError, match="foreach"):
        AdamW(p, foreach=True)
    for kw in ({"lr": -1.0}, {"eps": -1.0}, {"betas": (1.0, 0.9)}, {"betas": (0.9, -0.1)},
               {"weight_decay": -0.1}):
        with pytest.raises(ValueError):
            AdamW(p, **kw)
    with pytest.raises(NotImplementedError):
        AdamW(p, lr=torch.tensor(1e-3))
    with pytest.raises(ValueError):
        AdamW(p, chunk_elems=1000)


def test_at_most_16_param_groups():
    """One launch carries up to TM_MAX_GROUPS (16) hyper-parameter groups; more are refused
    at construction and by add_param_group, before any GPU work."""
    ps = [torch.nn.Parameter(torch.zeros(2)) for _ in range(17)]
    AdamW([{"params": [p]} for p in ps[:16]])
    with pytest.raises(ValueError, match="at most 16"):
        AdamW([{"params": [p]} for p in ps])
    opt = AdamW([{"params": [p]} for p in ps[:16]])
    with pytest.raises(ValueError, match="at most 16"):
        opt.add_param_group({"params": [ps[16]]})
    assert len(opt.param_groups) == 16  # the refused group was not added


def test_param_in_two_optimizers_has_no_single_owner():
    """A param held by two AdamW instances reads as unowned, so a clip over it scales in
    place (both optimizers see the scaled grads) instead of deferring into one of them."""
    from torchure_amd.optimizer.adamw import owner_of

    a, b = torch.nn.Parameter(torch.zeros(2)), torch.nn.Parameter(torch.zeros(2))
    o1 = AdamW([a, b])
    assert owner_of(a) is o1 and owner_of(b) is o1
    o2 = AdamW([b])
    assert owner_of(a) is o1 and owner_of(b) is None
    AdamW([b])
    assert owner_of(b) is None  # stays shared
    del o1
    import gc
    gc.collect()
    c = torch.nn.Parameter(torch.zeros(2))
    o3 = AdamW([a, c])  # a's previous owner is gone: o3 owns it
    assert owner_of(a) is o3 and owner_of(c) is o3 and o2 is not None


def test_owned_params_pickle_and_copy():
    """Params of this AdamW pickle, save and deep-copy as with torch's optimizers (the owner
    mark is not carried over: the saved or copied param belongs to no optimizer)."""
    import copy
    import io
    import pickle

    from torchure_amd.optimizer.adamw import owner_of

    m = torch.nn.Linear(4, 3)
    opt = AdamW(m.parameters())
    buf = io.BytesIO()
    torch.save(m, buf)
    buf.seek(0)
    m2 = torch.load(buf, weights_only=False)  # a file this test wrote
    assert torch.equal(m2.weight, m.weight) and owner_of(m2.weight) is None
    w = pickle.loads(pickle.dumps(m.weight))
    assert torch.equal(w, m.weight) and owner_of(w) is None
    t = m.weight.detach().clone()
    t._tm_owner = m.weight._tm_owner
    assert owner_of(copy.deepcopy(t)) is None  # (a shallow copy shares the mark, as it shares all attributes)
    assert owner_of(m.weight) is opt
    # the optimizer itself: its settings survive, and it owns the params it comes back with
    o = AdamW(m.parameters(), chunk_elems=4096, defer_clip=False)
    for o2 in (pickle.loads(pickle.dumps(o)), copy.deepcopy(o)):
        assert (o2.chunk_elems, o2.defer_clip) == (4096, False)
        assert all(owner_of(p) is o2 for g in o2.param_groups for p in g["params"])
        assert o2.param_groups[0]["params"][0] is not m.weight


def test_param_groups_have_torch_adamw_keys():
    m1, m2 = _model(), _model()
    mine = build_optimizer(m1, "adamw", {"lr": 3e-4, "weight_decay": 0.1, "betas": [0.9, 0.95], "fused": True})
    groups = [
        {"params": [p for p in m2.parameters() if p.dim() >= 2], "weight_decay": 0.1},
        {"params": [p for p in m2.parameters() if p.dim() < 2], "weight_decay": 0.0},
    ]
    ref = torch.optim.AdamW(groups, lr=3e-4, betas=[0.9, 0.95], fused=True)
    a, b = mine.state_dict(), ref.state_dict()
    assert [sorted(g) for g in a["param_groups"]] == [sorted(g) for g in b["param_groups"]]
    for ga, gb in zip(a["param_groups"], b["param_groups"]):
        for k in gb:
            if k != "betas":
                assert ga[k] == gb[k], k
        assert tuple(ga["betas"]) == tuple(gb["betas"])
    # builder.py:37-43 split: 2-D weights decay, biases / norm weights do not
    assert [len(g["params"]) for g in mine.param_groups] == [2, 3]
    assert [g["weight_decay"] for g in mine.param_groups] == [0.1, 0.0]


def test_load_torch_cpu_state_dict():
    """A checkpoint of torch.optim.AdamW (what torchure's Checkpointer saves)
    loads into the drop-in with identical state tensors and groups, except that the
    groups say fused (and foreach None), which is what this optimizer runs."""
    m = _model()
    ref = torch.optim.AdamW(m.parameters(), lr=1e-3)
    for _ in range(3):
        m(torch.randn(5, 8)).sum().backward()
        ref.step()
        ref.zero_grad()
    sd = ref.state_dict()
    mine = AdamW(m.parameters(), lr=1e-3)
    mine.load_state_dict(sd)
    got = mine.state_dict()
    assert got["param_groups"] == [dict(g, fused=True, foreach=None) for g in sd["param_groups"]]
    for k in sd["state"]:
        for key in ("step", "exp_avg", "exp_avg_sq"):
            assert torch.equal(got["state"][k][key], sd["state"][k][key])


def test_step_on_cpu_params_fails_loudly():
    m = _model()
    opt = AdamW(m.parameters())
    m(torch.randn(2, 8)).sum().backward()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()


def test_clip_errors():
    with pytest.raises(AssertionError):
        ta.clip_grad_norm([torch.nn.Parameter(torch.zeros(4))], None, 1.0)
    p = torch.nn.Parameter(torch.zeros(4))
    p.grad = torch.ones(4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ta.clip_grad_norm([p], None, 1.0)
    with pytest.raises(NotImplementedError):
        ta.clip_grad_norm([p], None, 1.0, shard_dims=("dp",))

    class Mesh:  # the MeshLike surface clip_grad_norm reads (torchure/core/collective.py:66-85)
        def __init__(self, sizes):
            self.sizes = sizes

        def size(self, dim):
            return self.sizes[dim]

    # a shard dimension with more than one rank needs a collective: rejected before any work
    with pytest.raises(NotImplementedError, match="'fsdp' has 2 ranks"):
        ta.clip_grad_norm([p], Mesh({"dp": 1, "fsdp": 2}), 1.0, shard_dims=("dp", "fsdp"))
    # size-1 dimensions pass the check and reach the device path (no GPU here)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ta.clip_grad_norm([p], Mesh({"dp": 1}), 1.0, shard_dims=("dp",))


def test_wsd_scheduler_matches_closed_form():
    m = _model()
    opt = AdamW(m.parameters(), lr=3e-4)
    sched = build_scheduler(opt, {"type": "wsd", "total_steps": 100, "warmup_ratio": 0.05, "decay_ratio": 0.2})
    for k in range(130):
        want = 3e-4 * oracle.wsd_scale(k, 100, 0.05, 0.2)
        assert opt.param_groups[0]["lr"] == want, k
        assert opt.param_groups[1 if len(opt.param_groups) > 1 else 0]["lr"] == want
        assert wsd_scale(k, 100, 0.05, 0.2) == oracle.wsd_scale(k, 100, 0.05, 0.2)
        sched.step()
    assert opt.param_groups[0]["initial_lr"] == 3e-4


def test_scheduler_state_roundtrip():
    m = _model()
    opt = AdamW(m.parameters(), lr=3e-4)
    s1 = build_scheduler(opt, {"type": "wsd", "total_steps": 50, "warmup_ratio": 0.1, "decay_ratio": 0.2})
    for _ in range(17):
        s1.step()
    opt2 = AdamW(m.parameters(), lr=3e-4)
    s2 = build_scheduler(opt2, {"type": "wsd", "total_steps": 50, "warmup_ratio": 0.1, "decay_ratio": 0.2})
    s2.load_state_dict(s1.state_dict())
    assert s2.last_epoch == 17 and s2.get_last_lr() == s1.get_last_lr()


def test_cosine_is_refused():
    opt = AdamW(_model().parameters())
    with pytest.raises(NotImplementedError):
        build_scheduler(opt, {"type": "cosine", "total_steps": 10, "warmup_ratio": 0.1, "decay_phase": 0.1,
                              "last_epoch": -1})


def test_sgd_registry_entry_passes_through():
    opt = build_optimizer(_model(), "sgd", {"lr": 0.1, "weight_decay": 0.0})
    assert isinstance(opt, torch.optim.SGD)


def test_fused_linear_ce_fails_loudly_without_gpu():
    from torchure_amd.loss import fused_linear_cross_entropy

    hidden = torch.randn(8, 4).to(torch.bfloat16)
    weight = torch.randn(16, 4)
    labels = torch.zeros(8, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fused_linear_cross_entropy(hidden, weight, labels)


def test_fused_linear_ce_chunk_sizing():
    from torchure_amd.loss.fused_linear_ce import auto_chunk_rows

    # 4 GiB of bf16 logits for the Qwen3 vocabulary: 14,080 rows (a multiple of 256)
    assert auto_chunk_rows(100000, 151936) == 14080
    assert auto_chunk_rows(8192, 151936) == 8192  # 8K tokens fit in one chunk
    assert auto_chunk_rows(10, 151936) == 10
    assert auto_chunk_rows(100000, 10 ** 9) == 256  # never below 256 rows


def test_host_list_primitives():
    """The C++ list walks of the step's host path, on CPU tensors (no GPU work)."""
    import numpy as np

    from torchure_amd import _native

    h = _native.host()
    ps = [torch.nn.Parameter(torch.zeros(3)) for _ in range(4)]
    ws = [None, torch.zeros(3, dtype=torch.bfloat16).requires_grad_(), None,
          torch.zeros(3, dtype=torch.bfloat16).requires_grad_()]
    ps[0].grad = torch.ones(3)
    ws[1].grad = torch.ones(3, dtype=torch.bfloat16)
    ps[3].grad = torch.ones(3)  # the master's own grad wins over the working copy's
    ws[3].grad = torch.ones(3, dtype=torch.bfloat16)
    gs, src = h.grads(ps, ws)
    assert src == bytes([1, 2, 0, 1])
    assert gs[0] is ps[0].grad and gs[1] is ws[1].grad and gs[2] is None and gs[3] is ps[3].grad
    assert list(h.ptrs([ps[0], None])) == [ps[0].data_ptr(), 0]
    v0 = [p._version for p in ps]
    h.bump(ps[:2])
    assert [p._version for p in ps] == [v0[0] + 1, v0[1] + 1, v0[2], v0[3]]
    assert list(h.versions([ps[0], None])) == [ps[0]._version, -1]
    assert h.version_sum(ps) == sum(p._version for p in ps)
    assert h.dense_contiguous(ps) and not h.dense_contiguous([torch.zeros(3, 4).t()])
    assert not h.dense_contiguous([None]) and not h.dense_contiguous([torch.zeros(2, 2).to_sparse()])
    assert h.same(ps, list(ps)) and not h.same(ps, ps[::-1]) and not h.same(ps, ps[:3])
    ptr, numel, code = h.grad_fields([torch.zeros(5)])
    assert numel[0] == 5 and code[0] == 255  # CPU tensors are not grad-table material
    _, _, code = h.grad_fields([torch.zeros(5, 2).to_sparse()])  # no storage: reported, not raised
    assert code[0] == 255
    from collections import defaultdict
    st = defaultdict(dict)
    st[ps[0]] = {"exp_avg": ps[1], "exp_avg_sq": ps[2], "step": ps[3]}
    sd = [st[ps[0]]]
    assert h.states_same(st, [ps[0]], sd, [ps[1]], [ps[2]], [ps[3]])
    assert not h.states_same(st, [ps[0]], sd, [ps[1]], [ps[3]], [ps[3]])  # another tensor
    assert not h.states_same(st, [ps[1]], sd, [ps[1]], [ps[2]], [ps[3]])  # no entry: no factory run
    assert ps[1] not in st
    ps[0]._tm_working = ws[1]
    assert h.attrs_same(ps[:2], "_tm_working", [ws[1], None])
    assert not h.attrs_same(ps[:2], "_tm_working", [None, None])
    with pytest.raises(TypeError):
        h.ptrs([1])
    assert isinstance(ptr, np.ndarray)


def test_shard_shapes_split_dim0_like_torch_chunk():
    """One rank's share of a dim-0 sharded parameter set has torch.chunk's pieces (FSDP2's
    Shard(0)): the ranks' shares put together are the whole set, rank 0 of the 4B set over 8
    ranks holds 502,808,512 params, and ranks past the last non-empty piece hold nothing."""
    from torchure_amd.workloads import numel, shapes_for, shard_shapes

    full = shapes_for("qwen3-4b")
    for ranks in (1, 3, 8):
        shares = [shard_shapes(full, ranks, r) for r in range(ranks)]
        assert sum(numel(s) for sh in shares for s in sh) == sum(numel(s) for s in full)
        for shape in set(full) | {(3, 5), (130,)}:
            want = [t.shape[0] for t in torch.zeros(shape[0]).chunk(ranks)]
            want += [0] * (ranks - len(want))
            got = [sum(s[0] for s in shard_shapes([shape], ranks, r)) for r in range(ranks)]
            assert got == want, (shape, ranks, got, want)
    r0 = shapes_for("qwen3-4b-shard8")
    assert r0 == shard_shapes(full, 8, 0) and sum(numel(s) for s in r0) == 502_808_512
    assert shard_shapes([(3, 5)], 8, 7) == [] and shard_shapes([(3, 5)], 8, 1) == [(1, 5)]
    with pytest.raises(ValueError):
        shard_shapes(full, 8, 8)


def test_bench_ddp_bucket_layout():
    """bench.py's DDP bucket leg lays grads out as torchure's DDP does
    (torchure/parallelism/data_parallel.py:86-105): reverse parameter order, a bucket closes
    before the param that would push it past the cap, and only multi-param buckets get a
    flat buffer whose views become the grads (values kept)."""
    import bench

    sizes = [100_000, 200_000, 50_000, 300_000, 10_000]  # fp32: 0.4, 0.8, 0.2, 1.2, 0.04 MB
    ps = [torch.nn.Parameter(torch.zeros(n)) for n in sizes]
    for i, p in enumerate(ps):
        p.grad = torch.full((p.numel(),), float(i))
    own = [p.grad for p in ps]
    # reversed: [10k] | [300k] | [50k, 200k] (1,000,000 B <= 1 MiB) | [100k]
    assert bench.ddp_bucket_grads(ps, bucket_mb=1) == 4
    for i in (0, 3, 4):
        assert ps[i].grad is own[i]
    g50, g200 = ps[2].grad, ps[1].grad
    assert g50.untyped_storage().data_ptr() == g200.untyped_storage().data_ptr()
    assert g200.data_ptr() == g50.data_ptr() + 4 * 50_000
    assert torch.equal(g50, torch.full((50_000,), 2.0)) and torch.equal(g200, torch.full((200_000,), 1.0))


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with a message: this build has no cross-GPU path."""
    import subprocess
    import sys as _sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = subprocess.run([_sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=root)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr and not p.stdout.strip()


def test_fused_linear_ce_default_chunk_is_the_reference_1024():
    """fused_linear_cross_entropy keeps the reference's default chunk_size=1024
    (torchure/loss/fused_linear_ce.py:131); None and "auto" opt into MI355X sizing."""
    import inspect

    from torchure_amd.loss import fused_linear_cross_entropy

    assert inspect.signature(fused_linear_cross_entropy).parameters["chunk_size"].default == 1024


def test_bench_cpu_baseline_on_a_small_set():
    """bench.py's CPU baseline times the reference composition over a whole parameter set
    with one thread per usable logical CPU, and reports the other sets under configs."""
    import bench

    out = bench.run_cpu_baseline(["tiny", "tiny"], steps=2, seconds=0.0)
    logical, physical = bench._cpu_topology()
    assert out["kind"] == "reference" and out["unit"] == "GB/s" and out["value"] > 0
    assert out["cores"] == out["logical_cpus"] == logical >= 1
    assert physical is None or 1 <= physical <= logical
    assert out["ms_per_step"] > 0 and "whole parameter set (24 tensors, 2622976 params)" in out["sample"]
    assert out["configs"]["tiny"]["n_params"] == 2622976


def test_fused_ce_grad_h_gemm_choice():
    """Chunks whose grad_h runs on the split-K MFMA GEMM: shapes it tiles (rows and hidden
    size multiples of 256, vocabulary of 64), except more than 64 output tiles of 256 x 256
    with a power-of-two hidden size, where the library GEMM measured faster; everything else
    stays on torch.matmul."""
    from torchure_amd.loss.fused_linear_ce import splitk_grad_h_fits

    v = 151936
    assert splitk_grad_h_fits(1024, 1024, v)  # the reference's chunk on the Qwen3-0.6B head
    assert splitk_grad_h_fits(4096, 1024, v)  # the trainer's chunk: 64 tiles
    assert not splitk_grad_h_fits(8192, 1024, v)  # 128 tiles
    assert splitk_grad_h_fits(1024, 4096, v) and not splitk_grad_h_fits(2048, 4096, v)
    assert splitk_grad_h_fits(2048, 2048, v) and not splitk_grad_h_fits(4096, 2048, v)
    # Qwen3-4B (2560) and 14B/32B (5120) heads: split-K at every chunk size
    assert splitk_grad_h_fits(4096, 2560, v) and splitk_grad_h_fits(8192, 2560, v)
    assert splitk_grad_h_fits(8192, 5120, v) and splitk_grad_h_fits(32768, 2560, v)
    assert not splitk_grad_h_fits(1000, 1024, v) and not splitk_grad_h_fits(1024, 1000, v)
    assert not splitk_grad_h_fits(1024, 1024, 151937) and not splitk_grad_h_fits(0, 1024, v)


def test_working_copy_freshness_rule():
    """``current_copy`` hands out an attached bf16 copy only while it still holds RNE(master):
    an in-place change of the master or of the copy itself (seen through their autograd
    version counters) makes readers cast the master again."""
    from torchure_amd.optimizer.working import current_copy, mark_current

    p = torch.randn(8, 4)
    w = p.to(torch.bfloat16)
    assert current_copy(p) is None  # nothing attached
    p._tm_working = w
    assert current_copy(p) is None  # attached but never marked
    mark_current(p, w)
    assert current_copy(p) is w
    w.add_(1)  # the copy written outside attach / refresh / step
    assert current_copy(p) is None
    w.copy_(p)
    mark_current(p, w)
    assert current_copy(p) is w
    p.mul_(2)  # the master changed: the copy is stale
    assert current_copy(p) is None
    mark_current(p, w)
    p2 = p.detach().clone()
    p2._tm_working = w.view(4, 8)  # wrong shape
    mark_current(p2, p2._tm_working)
    assert current_copy(p2) is None
    p3 = p.double()
    p3._tm_working = w
    assert current_copy(p3) is None  # not an fp32 master


def test_host_version_stamps_follow_shared_counters():
    """``stamp`` records each master's and copy's current autograd version on the copy and
    ``stamped`` compares them again; masters that are views of one buffer share one counter,
    so bumping all of them raises each one's version by their number, and the stamps taken
    after the bumps (what the step does) still match."""
    from torchure_amd import _native
    from torchure_amd.optimizer.working import current_copy

    h = _native.host()
    pool = torch.zeros(12)
    ps = [torch.nn.Parameter(pool[4 * i: 4 * i + 4]) for i in range(3)]
    cpool = torch.zeros(12, dtype=torch.bfloat16)
    ws = [cpool[4 * i: 4 * i + 4] for i in range(3)]
    for p, w in zip(ps, ws):
        p._tm_working = w
    assert not h.stamped(ps, ws)  # never stamped
    h.stamp(ps, ws)
    assert h.stamped(ps, ws)
    assert all(w._tm_master_version == p._version and w._tm_copy_version == w._version
               for p, w in zip(ps, ws))
    assert all(current_copy(p) is w for p, w in zip(ps, ws))
    v0 = ps[0]._version
    h.bump(ps + ws)  # what a step does after writing masters and copies
    assert ps[0]._version == v0 + 3 and ps[2]._version == v0 + 3  # one counter for the pool
    assert not h.stamped(ps, ws)
    h.stamp(ps, ws)
    assert h.stamped(ps, ws) and all(current_copy(p) is w for p, w in zip(ps, ws))
    with torch.no_grad():
        ps[1].add_(1)  # any in-place write into the pool makes every copy of it stale
    assert not h.stamped(ps, ws) and current_copy(ps[0]) is None
    with pytest.raises(ValueError):
        h.stamp(ps, ws[:2])


def test_fused_ce_calls_are_ordered_per_device():
    """CallOrder (torchure_amd/loss/fused_linear_ce.py) with stand-in streams and events: the
    first call on a device waits for nothing; a call on another stream waits for the event
    recorded at the end of the previous call on that device (and on no other device's); a
    call on the same stream as the previous one adds no wait; every call records its event
    after its work; a call that raises still records it. Also that the op holds its ordering
    lock while the host issues a call's work, so two host threads cannot interleave calls."""
    from torchure_amd.loss.fused_linear_ce import CallOrder

    log = []

    class Ev:
        n = 0

        def __init__(self):
            Ev.n += 1
            self.name = f"e{Ev.n}"

        def record(self, stream):
            log.append(("record", stream.name, self.name))

    class St:
        def __init__(self, name):
            self.name = name

        def wait_event(self, ev):
            log.append(("wait", self.name, ev.name))

        def __eq__(self, other):
            return isinstance(other, St) and other.name == self.name

        def __ne__(self, other):
            return not self == other

        def __hash__(self):
            return hash(self.name)

    cur = {"s": St("A")}
    order = CallOrder(current_stream=lambda dev: cur["s"], make_event=Ev)
    d0, d1 = torch.device("cuda", 0), torch.device("cuda", 1)

    def call(dev, stream, fail=False):
        cur["s"] = St(stream)
        with order.call(dev) as s:
            assert s.name == stream
            log.append(("work", stream))
            if fail:
                raise ValueError("planted")

    call(d0, "A")
    assert log == [("work", "A"), ("record", "A", "e1")]
    log.clear()
    call(d0, "B")  # another stream: waits for the previous call's end event
    assert log == [("wait", "B", "e1"), ("work", "B"), ("record", "B", "e2")]
    log.clear()
    call(d0, "B")  # same stream: in order already, no wait
    assert log == [("work", "B"), ("record", "B", "e3")]
    log.clear()
    call(d1, "C")  # another device: nothing to wait for
    assert log == [("work", "C"), ("record", "C", "e4")]
    log.clear()
    with pytest.raises(ValueError, match="planted"):
        call(d0, "A", fail=True)
    assert log == [("wait", "A", "e3"), ("work", "A"), ("record", "A", "e5")]
    log.clear()
    call(d0, "C")  # waits for the failed call's event, not an older one
    assert log[0] == ("wait", "C", "e5")
    log.clear()
    with order.call(torch.device("cpu")) as s:  # no GPU: nothing to order (the op raises later)
        assert s is None
    assert log == []

    # the lock is held while a call issues its work: another thread's call waits for it
    import threading

    inside = threading.Event()
    release = threading.Event()
    seen = []

    def first():
        with order.call(d0):
            inside.set()
            release.wait(10)
            seen.append("first done")

    def second():
        inside.wait(10)
        with order.call(d0):
            seen.append("second")

    t1, t2 = threading.Thread(target=first), threading.Thread(target=second)
    t1.start()
    t2.start()
    inside.wait(10)
    t2.join(0.2)
    assert seen == [] and t2.is_alive()
    release.set()
    t1.join(10)
    t2.join(10)
    assert seen == ["first done", "second"]


def test_update_shifted_grid_covers_every_element_once():
    """The update kernel's slice rules (torchure_amd/csrc/tm_optim.hip, adamw_update_kernel and
    slice_of), restated in numpy: with chunks of C elements cut into C / 256 one-wave slices,
    slice s of chunk c starting at start = c*C + 256*s, and a tensor of n elements at grid phase
    ph (a multiple of 4 below 256), the wave returns when start - ph >= n and start > 0; lane t
    takes e = start + 4t - ph, wrapped by ceil(n/C)*C when negative; it updates [e, e+4) when
    e + 4 <= n, else [e, n) element by element when e < n. Every element of [0, n) must be
    updated exactly once, every group of 4 must start 16-byte aligned in arrays at that phase
    ((e + ph) % 4 == 0), and only the last group of the tensor may be partial. Lengths around
    the chunk boundaries (1..3C+300 at C = 2048, around k*C at C = 4096 and 16,384) and every
    phase 0..252."""
    import numpy as np

    def check(n, C):
        n_chunks = -(-n // C)
        spc = C // 256
        start = (np.arange(n_chunks)[:, None] * C + np.arange(spc)[None, :] * 256).reshape(-1)
        phs = np.arange(0, 256, 4)
        lanes = np.arange(64) * 4
        # (phase, slice, lane)
        st = np.broadcast_to(start[None, :, None], (phs.size, start.size, 64))
        ph = np.broadcast_to(phs[:, None, None], st.shape)
        alive = ~((st - ph >= n) & (st > 0))
        e = st + lanes[None, None, :] - ph
        e = np.where(e < 0, e + n_chunks * C, e)
        full = alive & (e + 4 <= n)
        tail = alive & (e < n) & ~full
        assert not np.any(full & ((e + ph) % 4 != 0)), (n, C)
        assert np.all(e[tail] + 4 > n), (n, C)
        counts = np.zeros((phs.size, n), dtype=np.int64)
        pidx = np.broadcast_to(np.arange(phs.size)[:, None, None], st.shape)
        for j in range(4):
            m = (full | tail) & (e + j < n)
            np.add.at(counts, (pidx[m], e[m] + j), 1)
        assert np.all(counts == 1), (n, C, np.argwhere(counts != 1)[:4])

    for n in range(1, 3 * 2048 + 301, 7):
        check(n, 2048)
    for n in list(range(1, 40)) + [2047, 2048, 2049, 6143, 6144, 6145]:
        check(n, 2048)
    for C in (4096, 16384):
        for k in (1, 2, 3):
            for n in range(k * C - 260, k * C + 261, 13):
                check(n, C)


def test_pooled_state_layout(tmp_path):
    """pooled_layout / pooled_moments (torchure_amd/optimizer/adamw.py): views never overlap and
    stay inside the pool; every view starts 16-byte aligned; a tensor given a phase starts that
    many elements past a 1 KiB boundary of the pool (so a param's moments share its master's
    phase); the two roles share one layout; Qwen3 sets with 1 KiB-aligned masters need no
    padding; random phases need little; and torch.save of pooled moments is not larger than of
    the same moments as separate tensors."""
    import numpy as np

    from torchure_amd.optimizer.adamw import master_phase, pooled_layout, pooled_moments
    from torchure_amd.workloads import shapes_for

    rng = np.random.default_rng(5)
    numels = [int(x) for x in rng.integers(0, 5000, 300)] + [256, 512, 128, 1, 3, 4, 0, 1024 * 1024]
    for phases in (None, [int(x) * 4 for x in rng.integers(0, 64, len(numels))],
                   [None if k % 5 == 0 else 128 * (k % 2) for k in range(len(numels))]):
        offs, total = pooled_layout(numels, phases)
        spans = sorted((o, o + n) for o, n in zip(offs, numels) if n)
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])) and spans[-1][1] <= total
        assert all(o % 4 == 0 for o in offs)
        want = phases if phases is not None else [0 if n % 256 == 0 else None for n in numels]
        assert all(ph is None or o % 256 == ph for o, ph in zip(offs, want))
        assert total <= sum((n + 3) // 4 * 4 for n in numels) + 256 * len(numels)
    for cfg in ("tiny", "qwen3-0.6b", "qwen3-4b"):
        ns = [int(np.prod(s)) for s in shapes_for(cfg)]
        assert pooled_layout(ns, [0 if n >= 256 else None for n in ns])[1] == sum(ns)  # no padding
    ps = [torch.zeros(s) for s in [(3, 5), (256,), (7,), (2, 128), (64, 64), (1001,)]]
    views = pooled_moments(ps, zero=True)
    for p, m, v in views:
        assert m.shape == p.shape and v.shape == p.shape and m.dtype == torch.float32
        assert m.data_ptr() % 1024 == v.data_ptr() % 1024
        assert m.data_ptr() % 16 == 0 and not m.any()
        if master_phase(p) is not None and p.numel() >= 256:
            assert (m.data_ptr() // 4) % 256 == master_phase(p)
    assert len({m.untyped_storage().data_ptr() for _, m, _ in views}) == 1
    # torch.save writes a pool once (one record per storage): with no padding, as for Qwen3 sets
    # on 1 KiB-aligned masters, the file is not larger than with one tensor per moment
    ns = [int(np.prod(s)) for s in shapes_for("tiny")]
    offs, total = pooled_layout(ns, [0 if n >= 256 else None for n in ns])
    pools = torch.zeros(total), torch.zeros(total)
    state = {i: {"exp_avg": pools[0][o:o + n], "exp_avg_sq": pools[1][o:o + n]} for i, (o, n) in enumerate(zip(offs, ns))}
    torch.save(state, tmp_path / "pooled.pt")
    torch.save({i: {k: t.clone() for k, t in st.items()} for i, st in state.items()}, tmp_path / "separate.pt")
    assert os.path.getsize(tmp_path / "pooled.pt") <= os.path.getsize(tmp_path / "separate.pt")
