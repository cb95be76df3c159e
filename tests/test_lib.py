"""The C-ABI library loads and exports every entry point include/ress_hip.h declares, with
the argument counts the ctypes binding uses. CPU only (no kernel is launched)."""

import ctypes
import os
import re

import pytest

from ress_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ress_hip.h")


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[a-z ]+\*?\s*(ress_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return decls


@pytest.fixture(scope="module")
def library():
    if not os.path.exists(_lib.LIB_PATH):
        from ress_amd.build import build_library
        build_library()
    return _lib.lib()


def test_header_declares_entry_points():
    decls = _declarations()
    assert len(decls) >= 14
    assert "ress_sparse_attn_fwd" in decls and "ress_qattn_block_sparse_fwd" in decls


def test_every_declared_symbol_is_exported(library):
    for name in _declarations():
        assert hasattr(library, name), name
        assert isinstance(getattr(library, name), ctypes._CFuncPtr)


def test_binding_argument_counts_match_header(library):
    decls = _declarations()
    for name, sig in _lib._SIGS.items():
        assert name in decls, f"{name} bound but not declared"
        assert len(sig) == decls[name], (name, len(sig), decls[name])
    assert set(_lib.exported_symbols()) == set(decls)


def test_abi_version_and_error_string(library):
    assert library.ress_abi_version() == 5
    assert isinstance(library.ress_last_error(), bytes)


def test_workspace_sizes(library):
    # 256-byte schedule header + 8 XCD ranges x (split rows) x 3 parts x (O, m, l) of
    # 256 threads x (32 + 2) floats; split rows = min(32, query blocks incl. one per head)
    part = 3 * 256 * 34 * 4
    assert library.ress_attn_sched_bytes(1, 16, 21984) == 256 + 8 * 32 * part
    assert library.ress_attn_sched_bytes(2, 3, 0) == 256 + 8 * 6 * part
    assert library.ress_attn_sched_bytes(0, 3, 10) == -1
    # SpargeAttn mirror: status word (256 B), packed V (64x64 bf16 per key block), the checked
    # LUT and counts (each rounded to 256 B), then the attention's workspace
    assert library.ress_qattn_workspace_size(1, 2, 300, 200) == (256 + 2 * 4 * 4096 * 2 + 256 + 256 + 256
                                                                  + 8 * 8 * part)
    assert library.ress_qattn_workspace_size(1, 2, -1, 200) == -1


def test_argument_validation_without_a_gpu(library):
    # bad geometry is rejected on the host before any launch
    rc = library.ress_pooled_scores(None, None, 0, 0, 0, 0, ctypes.c_float(0.125), None, None, None)
    assert rc == -1
    assert b"bad geometry" in library.ress_last_error()
    rc = library.ress_baseline_budget(None, 4, 10, ctypes.c_float(-1.0), -1, None, None)
    assert rc == -1 and b"at least one" in library.ress_last_error()
    rc = library.ress_qattn_block_sparse_fwd(*([None] * 3), 0, None, 0, None, None, None, None, None, 1, 1, 128, 64,
                                             0, 0, 0, 0, 0, 0, 0, 0, 1, ctypes.c_float(0.125), 0, None, 0, None)
    assert rc == -1 and b"tensor_layout" in library.ress_last_error()


def test_attention_rejects_heads_beyond_the_descriptor_range(library):
    # the attention kernels address a head's K/V blocks (8 KiB each) through buffer descriptors
    # with a 32-bit size: a sequence of more than 2^31 / 8192 key blocks is refused on the host,
    # before any pointer is used (the fake, aligned addresses below are never dereferenced)
    fake = ctypes.c_void_p(4096)
    frames, P, S = 12300, 1374, 5  # 16.9 M keys: 264,070 blocks of 64
    args = (fake, 0, 0, 64, fake, fake, fake, fake, fake, 1, 1, frames, P, S, None, ctypes.c_float(0.125), fake, 0,
            0, 0, 64, fake, None)
    assert library.ress_sparse_attn_fwd_f16(*args) == -1
    assert b"2 GiB" in library.ress_last_error()
