"""The C-ABI library loads, exports every declared symbol, and validates its
arguments on the host (no compute calls: these run without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mi355x_kernels.h"
LIB = ROOT / "torch-mojo-backend_amd" / "torch_mojo_backend" / "eager_kernels" / "libmi355x_kernels.so"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(mi355x_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def raw():
    if not LIB.exists():
        pytest.fail(f"{LIB} not built: run __graft_entry__.build()")
    return ctypes.CDLL(str(LIB))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    for name in ("mi355x_attn_fwd", "mi355x_attn_bwd", "mi355x_gemm", "mi355x_layer_norm_fwd",
                 "mi355x_layer_norm_bwd", "mi355x_gelu_fwd", "mi355x_gelu_bwd",
                 "mi355x_softmax_fwd", "mi355x_softmax_bwd", "mi355x_nll_fwd", "mi355x_nll_bwd",
                 "mi355x_embedding_fwd", "mi355x_embedding_bwd", "mi355x_fused_adamw",
                 "mi355x_foreach_norm", "mi355x_foreach_apply", "mi355x_copy", "mi355x_map"):
        assert name in syms


def test_library_exports_every_declared_symbol(raw):
    missing = [s for s in declared_symbols() if not hasattr(raw, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_loader_signatures_cover_the_header():
    from torch_mojo_backend.eager_kernels import SIGNATURES

    assert sorted(SIGNATURES) == declared_symbols()


def test_abi_version_and_target(raw):
    raw.mi355x_abi_version.restype = ctypes.c_int
    raw.mi355x_target.restype = ctypes.c_char_p
    from torch_mojo_backend.eager_kernels import ABI_VERSION

    assert raw.mi355x_abi_version() == ABI_VERSION
    assert raw.mi355x_target() == b"gfx950"


def test_library_matches_its_sources(raw):
    """The built library carries the digest of the sources it was built
    from, and the loader's digest of the tree agrees (a stale prebuilt .so
    would be refused with a rebuild message)."""
    from torch_mojo_backend.eager_kernels import _expected_source_hash

    raw.mi355x_source_hash.restype = ctypes.c_char_p
    built = raw.mi355x_source_hash().decode()
    assert built != "unknown" and built == _expected_source_hash()


def test_host_side_validation_reports_errors(raw):
    """Argument checks fail before any launch, with a message."""
    from torch_mojo_backend.eager_kernels import SIGNATURES

    fn = raw.mi355x_gemm
    fn.restype, fn.argtypes = SIGNATURES["mi355x_gemm"]
    raw.mi355x_last_error.restype = ctypes.c_char_p
    # unsupported dtype code 7 (int8)
    rc = fn(None, 0, 1, 0, None, 1, 1, 0, None, 1, 1, 0, 7, None, 0, 0, 1, 4, 4, 4, None, 0, None)
    assert rc == 1
    assert b"unsupported dtype" in raw.mi355x_last_error()
    # A with neither a unit row nor column stride
    rc = fn(None, 1, 4, 0, None, 8, 2, 0, None, 1, 4, 0, 1, None, 0, 0, 1, 4, 4, 4, None, 0, None)
    assert rc == 1
    assert b"unit row or column stride" in raw.mi355x_last_error()
    att = raw.mi355x_attn_fwd
    att.restype, att.argtypes = SIGNATURES["mi355x_attn_fwd"]
    s = (ctypes.c_int64 * 3)(0, 0, 0)
    rc = att(None, s, None, None, s, None, s, None, s, 1, 1, 8, 8, 48, 0.1, 1, 1, None)
    assert rc == 3  # head_dim 48 unsupported
    assert b"head_dim" in raw.mi355x_last_error()


def test_workspace_queries_are_host_only(raw):
    from torch_mojo_backend.eager_kernels import SIGNATURES

    for name in ("mi355x_layer_norm_bwd_workspace_bytes", "mi355x_attn_bwd_workspace_bytes",
                 "mi355x_embedding_bwd_workspace_bytes", "mi355x_reduce_workspace_bytes"):
        getattr(raw, name).restype, getattr(raw, name).argtypes = SIGNATURES[name]
    assert raw.mi355x_layer_norm_bwd_workspace_bytes(16384, 768) == 2 * 256 * 768 * 4  # 256 block partials of dgamma and dbeta
    assert raw.mi355x_attn_bwd_workspace_bytes(8, 12, 1024, 1024, 64) >= 8 * 12 * 1024 * 4
    assert raw.mi355x_embedding_bwd_workspace_bytes(16384, 50257) >= 16384 * 16
    assert raw.mi355x_reduce_workspace_bytes(1, 1 << 20, 1) > 0
    assert raw.mi355x_reduce_workspace_bytes(16384, 768, 1) == 0
