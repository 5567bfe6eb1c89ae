"""The C-ABI library loads and exports every entry point include/moe_prefetch.h
declares, with the ctypes signatures matching the header (CPU only; no call
here touches a GPU)."""
import os
import re

import moe_prefetch
from moe_prefetch import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "moe_prefetch.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = header_functions()
    for must in ("moe_memcpy_h2d_batch", "moe_cache_create", "moe_cache_observe", "moe_cache_step",
                 "moe_route", "moe_experts", "moe_decode_token", "moe_pool_copy"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = moe_prefetch.lib()
    missing = [n for n in header_functions() if not hasattr(L, n)]
    assert missing == []


def test_ctypes_table_covers_header():
    assert set(header_functions()) == set(_lib.SIGNATURES)


def test_pure_host_queries():
    L = moe_prefetch.lib()
    assert L.moe_abi_version() == 1
    assert L.moe_expert_bytes(2048, 768, _lib.TYPE_Q4K) == 2654208
    assert L.moe_expert_bytes(2048, 768, _lib.TYPE_Q6K) == 3059712
    assert L.moe_expert_bytes(2048, 512, _lib.TYPE_Q4K) == 1769472
    assert L.moe_expert_bytes(2048, 512, _lib.TYPE_Q6K) == 2039808
    assert L.moe_route_workspace_bytes(128, 1) > 0
    assert L.moe_experts_workspace_bytes(768, 8) >= 8 * 768 * 4


def test_h2d_batch_refuses_on_the_host():
    # the reference's contract (patches/0006...:52-76): n <= 0 is done at once;
    # a batch that cannot be copied returns false and the caller treats it as
    # not done.  Null arrays or slice addresses are refused before any copy.
    import ctypes
    L = moe_prefetch.lib()
    assert L.moe_memcpy_h2d_batch(0, None, None, None, 0) is True
    assert L.moe_memcpy_h2d_batch(0, None, None, None, -3) is True
    assert L.moe_memcpy_h2d_batch(0, None, None, None, 2) is False
    P = ctypes.c_void_p * 2
    buf = ctypes.create_string_buffer(64)
    dst, src = P(ctypes.addressof(buf), None), P(ctypes.addressof(buf), ctypes.addressof(buf))
    sizes = (ctypes.c_size_t * 2)(16, 16)
    assert L.moe_memcpy_h2d_batch(0, dst, src, sizes, 2) is False
    assert b"slice 1 of 2" in L.moe_last_error()


def test_static_scratch_size_matches_header():
    text = open(os.path.join(ROOT, "include", "moe_prefetch.h")).read()
    m = re.search(r"#define MOE_GROUPED_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.GROUPED_STATIC_SCRATCH_BYTES
