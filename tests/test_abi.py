"""CPU: the C-ABI library builds, loads and exports exactly what include/*.h declares.

No kernel is launched here (no GPU in CI); entry points are only called with
arguments the library rejects on the host, before any HIP call.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from flexengine_amd import _lib

REPO = Path(__file__).resolve().parent.parent
HEADERS = sorted((REPO / "include").glob("*.h"))


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(fe_[a-z0-9_]+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from flexengine_amd import build
        build.build()
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    decl = declared_functions()
    assert decl, "no declarations found"
    for name in decl:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (fe_[a-z0-9_]+)", out))
    assert exported == decl, f"exported-only {exported - decl}, declared-only {decl - exported}"


def test_python_signatures_cover_the_header():
    assert set(_lib.SIGNATURES) == declared_functions()


def test_header_argument_counts_match_ctypes():
    text = "".join(re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S) for h in HEADERS)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text, flags=re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), f"{name}: header {len(params)} args, ctypes {len(args)}"


def test_version_and_error_strings(lib):
    assert lib.fe_version() >= 100
    for code in (_lib.FE_OK, _lib.FE_ERR_INVALID_ARGUMENT, _lib.FE_ERR_UNSUPPORTED, _lib.FE_ERR_WORKSPACE):
        assert _lib.error_string(code)
    assert "unsupported" in _lib.error_string(_lib.FE_ERR_UNSUPPORTED)


def test_host_side_validation_rejects_before_launch(lib):
    """Invalid configurations return an error code without touching the GPU."""
    null = None
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    # head_dim 1024 is past the generic kernel's 512
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 12, 2, 1024, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    # group size 129 > 128; group 67 (no divisor from 8 to 16) x head_dim 136 > 8192
    # elements (group 64 x 192 is taken: four virtual KV heads, padded to 256)
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 129, 1, 8, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 64, 1, 192, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 67, 1, 136, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    # the generic shapes (head_dim 96, group 32) take no plan; without one their null
    # pointers are the error
    rc = lib.fe_paged_decode_planned(null, 0, null, null, null, 0, null, null, 1, null, 1, null,
                                     null, 0, 1, 12, 2, 96, 16, 0.1, 0, fake, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 32, 1, 128, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    rc = lib.fe_prefill_paged(null, null, null, null, 1, null, 1, null, null, 1, 1, 1, 12, 2, 96,
                              16, 0.1, null, 0, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    rc = lib.fe_prefill_paged(null, null, null, null, 1, null, 1, null, null, 1, 1, 1, 2, 1, 520,
                              16, 0.1, null, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    # block size not a power of two
    rc = lib.fe_paged_decode(null, 0, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 12, 2, 128, 12, 0.1, 0, null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    # null pointers
    rc = lib.fe_paged_decode(null, 1536, null, null, null, 0, null, null, 1, null, 1, null, null, 0,
                             1, 12, 2, 128, 16, 0.1, 0, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    # Hq not a multiple of Hkv
    rc = lib.fe_prefill_paged(null, null, null, null, 1, null, 1, null, null, 1, 1, 1, 12, 5, 128, 16,
                              0.1, null, 0, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    rc = lib.fe_write_kv(null, null, 256, null, null, 4, null, null, 3, 2, 128, 16, null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    # shared-prefix decode: block size 8 cannot split at 16-token tiles; missing
    # group arrays; a negative group count
    fake = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.fe_paged_decode_shared_prefix(null, 1536, null, null, null, 0, null, null, 1, null, 1,
                                           null, fake, fake, 1, null, 0, 1, 12, 2, 128, 8, 0.1, 0,
                                           null)
    assert rc == _lib.FE_ERR_UNSUPPORTED
    rc = lib.fe_paged_decode_shared_prefix(null, 1536, null, null, null, 0, null, null, 1, null, 1,
                                           null, null, null, 1, null, 0, 1, 12, 2, 128, 16, 0.1, 0,
                                           null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    rc = lib.fe_paged_decode_shared_prefix(null, 1536, null, null, null, 0, null, null, 1, null, 1,
                                           null, null, null, -1, null, 0, 1, 12, 2, 128, 16, 0.1, 0,
                                           null)
    assert rc == _lib.FE_ERR_INVALID_ARGUMENT
    # empty work is a successful no-op
    assert lib.fe_write_kv(null, null, 256, null, null, 4, null, null, 0, 2, 128, 16, null) == 0
    assert lib.fe_lse_merge(null, null, 1, 0, 128, null, null, null) == 0
    assert lib.fe_lse_merge_bf16(null, null, 1, 0, 128, null, null, null) == 0


def test_workspace_size_grows_with_batch_and_target(lib):
    a = lib.fe_paged_decode_workspace_size(64, 12, 128, 4096, 0)
    b = lib.fe_paged_decode_workspace_size(128, 12, 128, 4096, 0)
    c = lib.fe_paged_decode_workspace_size(64, 12, 128, 4096, 2048)
    assert 0 < a < b and a < c
    assert a % 256 == 0
    assert lib.fe_paged_decode_workspace_size(-1, 12, 128, 4096, 0) == 0
    # prefill workspace: tickets only for big prefills, tickets + partials for small ones
    big = lib.fe_prefill_workspace_size(8, 8192, 12, 2, 128)
    small = lib.fe_prefill_workspace_size(4, 1377, 12, 2, 128)
    assert big >= 65536 * 4 and small > 65536 * 4
    assert lib.fe_prefill_workspace_size(1, 10, 12, 5, 128) == 0
    # the shared-prefix decode adds its prefix outputs (and key-split partials)
    sp = lib.fe_paged_decode_shared_prefix_workspace_size(256, 12, 2, 128, 4096, 8, 0)
    plain = lib.fe_paged_decode_workspace_size(256, 12, 128, 4096, 0)
    assert sp >= plain + 256 * 12 * 128 * 4 and sp % 256 == 0
    assert lib.fe_paged_decode_shared_prefix_workspace_size(256, 12, 5, 128, 4096, 8, 0) == 0
    # very long tables raise the split target (pieces stay <= 4096 keys)
    d = lib.fe_paged_decode_workspace_size(64, 12, 128, 1 << 20, 0)
    assert d > a


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libfe_paged.so")
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_cpu_tensors_are_rejected_not_computed():
    """The product path has no CPU fallback."""
    import torch
    from flexengine_amd import ops
    q = torch.zeros(1, 12, 128, dtype=torch.float16)
    pool = torch.zeros(2, 16, 2, 128, dtype=torch.float16)
    t = torch.zeros(1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.paged_decode(q, pool, pool, t, torch.ones(1, dtype=torch.int32))


def test_plan_error_word_constants_match_the_header():
    """ops.plan_error reads the words the header places; the kernels static_assert the same."""
    from flexengine_amd import ops
    text = (Path(__file__).resolve().parents[1] / "include" / "flexengine_amd.h").read_text()
    macros = dict(re.findall(r"#define\s+(FE_\w+)\s+(\d+)", text))
    assert int(macros["FE_DECODE_PLAN_ERROR_OFFSET"]) == ops._PLAN_ERROR_OFFSET["DecodePlan"]
    assert int(macros["FE_PREFILL_PLAN_ERROR_OFFSET"]) == ops._PLAN_ERROR_OFFSET["PrefillPlan"]
    assert int(macros["FE_PLAN_ERR_SIZES"]) == ops.PLAN_ERR_SIZES
    assert int(macros["FE_PLAN_ERR_STALE"]) == ops.PLAN_ERR_STALE
