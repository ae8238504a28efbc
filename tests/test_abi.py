"""The C-ABI library loads and exports everything include/torchure_amd.h declares.

No compute call needs a GPU here: only the host-side table helpers and the
argument validation, which return before any HIP call.
"""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from torchure_amd import _native


def _header() -> str:
    with open(_native.HEADER_PATH) as f:
        return f.read()


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", _header(), flags=re.S)
    return sorted(set(re.findall(r"\b(tm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared, "no tm_* functions parsed from the header"
    assert sorted(_native.EXPORTED) == declared


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_constants():
    h = _header()
    assert int(re.search(r"#define TM_ABI_VERSION (\d+)", h).group(1)) == _native.lib().tm_abi_version()
    for name in ("TM_GRAD_F32", "TM_FLAG_CLIP", "TM_MAX_GROUPS", "TM_CHUNK_ALIGN", "TM_NORM_PARTIALS",
                 "TM_NOALLOC_MAX_TENSORS"):
        val = int(re.search(rf"#define {name} (\d+)u?", h).group(1))
        assert getattr(_native, name) == val, name


def test_tensor_record_layout_matches_header():
    body = re.search(r"typedef struct tm_tensor \{(.*?)\} tm_tensor_t;", _header(), re.S).group(1)
    fields = re.findall(r"\b(?:uint64_t|int64_t|int32_t|uint32_t)\s+(\w+);", body)
    assert tuple(fields) == _native.TENSOR_DTYPE.names
    assert _native.TENSOR_DTYPE.itemsize == 64
    body = re.search(r"typedef struct tm_hyper \{(.*?)\} tm_hyper_t;", _header(), re.S).group(1)
    assert tuple(re.findall(r"double\s+(\w+);", body)) == tuple(f for f, _ in _native.TmHyper._fields_)


def test_chunk_table():
    numels = np.array([0, 1, 2048, 2049, 5000, 0, 4096], dtype=np.int64)
    t = _native.fill_chunks(numels, 2048)
    want = [(i, c) for i, n in enumerate(numels) for c in range(-(-int(n) // 2048))]
    assert [(int(a), int(b)) for a, b in zip(t["tensor"], t["chunk"])] == want
    assert len(_native.fill_chunks(np.zeros(3, np.int64), 2048)) == 0


def test_chunk_table_errors():
    lib = _native.lib()
    numels = np.array([5, -1], dtype=np.int64)
    assert lib.tm_count_chunks(numels.ctypes.data, 2, 2048) < 0
    assert b"negative numel" in lib.tm_last_error()
    ok = np.array([5000], dtype=np.int64)
    out = np.zeros(1, dtype=_native.CHUNK_DTYPE)
    assert lib.tm_fill_chunks(ok.ctypes.data, 1, 2048, out.ctypes.data, 1) < 0  # capacity too small


def test_workspace_bytes():
    a = _native.workspace_bytes(0)
    b = _native.workspace_bytes(1000)
    assert a >= 8 * _native.TM_NORM_PARTIALS and a % 256 == 0
    assert b - a >= 64 * 1000


def test_argument_validation_without_gpu():
    """Invalid arguments are rejected on the host before any HIP call."""
    lib = _native.lib()
    hyper = _native.hyper_array([(3e-4, 0.9, 0.95, 0.1, 1e-8)])
    fake = ctypes.c_void_p(0x1000)
    assert lib.tm_adamw_step(fake, 1, fake, 1, 2048, hyper, 0, None, fake, None) == _native.TM_OK - 1
    assert b"n_groups" in lib.tm_last_error()
    assert lib.tm_adamw_step(fake, 1, fake, 1, 1000, hyper, 1, None, fake, None) < 0
    assert b"chunk_elems" in lib.tm_last_error()
    assert lib.tm_grad_norm(fake, 1, fake, 1, 2048, 1.0, 1, None, fake, fake, None) < 0
    assert lib.tm_grad_norm(fake, 1, fake, 1, 2048, 1.0, 1, fake, fake, None, None) < 0
    assert lib.tm_grad_scale(fake, 1, fake, 1, 2048, None, None) < 0
    assert lib.tm_grad_accumulate_bf16(None, None, 10, None) < 0
    assert lib.tm_cast_bf16(None, None, -1, None) < 0
    assert lib.tm_grad_norm(None, 1, fake, 1, 2048, 1.0, 0, fake, fake, None, None) < 0
    # tm_stream_copy: size, alignment and overlap are checked before any launch
    assert lib.tm_stream_copy(ctypes.c_void_p(0x2000), fake, 24, None) < 0
    assert b"multiple of 16" in lib.tm_last_error()
    assert lib.tm_stream_copy(ctypes.c_void_p(0x2008), fake, 32, None) < 0
    assert b"aligned" in lib.tm_last_error()
    assert lib.tm_stream_copy(ctypes.c_void_p(0x1010), fake, 32, None) < 0
    assert b"overlap" in lib.tm_last_error()
    assert lib.tm_stream_copy(fake, fake, 0, None) == _native.TM_OK
    # the fused norm of the last micro-step needs one fp64 slot per 256-element slice (chunks
    # padded to 64 slots) beyond the 16 KB of block partials, and refuses less
    ws = lib.tm_accum_norm_workspace_bytes
    assert ws(10, 16384) == 16384 + 10 * 64 * 8
    assert ws(10, 2048) == 16384 + 10 * 64 * 8 and ws(3, 18432) == 16384 + 3 * 128 * 8
    assert ws(0, 16384) == 16384
    assert lib.tm_grad_accumulate_list(fake, 1, fake, 10, 16384, 1, fake, ws(10, 16384) - 8, fake, None) < 0
    assert b"needed" in lib.tm_last_error()
    assert lib.tm_grad_accumulate_list(fake, 1, fake, 1, 16384, 1, None, 1 << 20, fake, None) < 0


def test_grad_h_gemm_workspace_and_shape_checks_without_gpu():
    """The split-K grad_h GEMM: K splits picked by the launch's cost model, fp32 partials of
    rows x dim per split; shapes it does not tile, misaligned pointers and short workspaces are
    refused before any HIP call."""
    lib = _native.lib()
    ws = lib.tm_ce_grad_h_workspace_bytes
    v = 151936
    assert ws(1024, v, 1024) == 16 * 1024 * 1024 * 4  # 16 tiles x 16 splits: one round of 256 CUs
    assert ws(2048, v, 1024) == 8 * 2048 * 1024 * 4
    assert ws(4096, v, 1024) == 4 * 4096 * 1024 * 4
    assert ws(8192, v, 1024) == 2 * 8192 * 1024 * 4  # 128 tiles x 2 splits
    assert ws(1024, v, 2560) == 6 * 1024 * 2560 * 4  # 40 tiles x 6 splits: 240 workgroups
    assert ws(3072, v, 1024) == 16 * 3072 * 1024 * 4  # 48 x 16: three full rounds
    assert ws(8192, v, 4096) == 1 * 8192 * 4096 * 4  # 512 tiles fill two rounds by themselves
    assert ws(256, 640, 256) == 10 * 256 * 256 * 4  # 10 K slices: one per split
    assert ws(1000, v, 1024) == 0 and ws(1024, v, 1000) == 0 and ws(0, v, 256) == 0 and ws(256, 100, 256) == 0
    fake = ctypes.c_void_p(0x1000)
    big = 1 << 40
    for rows, vocab, dim in ((1000, 4096, 1024), (1024, 4000, 1024), (1024, 4096, 1000), (0, 4096, 256)):
        assert lib.tm_ce_grad_h_bf16(fake, fake, fake, rows, vocab, dim, fake, big, None) < 0
        assert b"multiples" in lib.tm_last_error()
    odd = ctypes.c_void_p(0x1008)
    assert lib.tm_ce_grad_h_bf16(fake, odd, fake, 256, 4096, 256, fake, big, None) < 0
    assert b"aligned" in lib.tm_last_error()
    assert lib.tm_ce_grad_h_bf16(fake, fake, fake, 256, 4096, 256, fake, ws(256, 4096, 256) - 1, None) < 0
    assert b"workspace" in lib.tm_last_error()
    assert lib.tm_ce_grad_h_bf16(fake, None, fake, 256, 4096, 256, fake, big, None) < 0


def test_grad_w_fold_argument_checks_without_gpu():
    """tm_ce_grad_w_fold takes 1 to 8 chunks, all non-null, and grad_out / n_valid both or
    neither; the checks run before any HIP call."""
    lib = _native.lib()
    fake = ctypes.c_void_p(0x1000)
    ptrs = (ctypes.c_void_p * 9)(*([0x1000] * 9))
    for k in (0, 9):
        assert lib.tm_ce_grad_w_fold(fake, ptrs, k, 100, 0, None, None, None) < 0
        assert b"chunks" in lib.tm_last_error()
    assert lib.tm_ce_grad_w_fold(fake, None, 2, 100, 0, None, None, None) < 0
    holes = (ctypes.c_void_p * 2)(0x1000, None)
    assert lib.tm_ce_grad_w_fold(fake, holes, 2, 100, 0, None, None, None) < 0
    assert b"null chunk 1" in lib.tm_last_error()
    assert lib.tm_ce_grad_w_fold(fake, ptrs, 2, 100, 0, fake, None, None) < 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(_native, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _native.lib()
