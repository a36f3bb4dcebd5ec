"""The C ABI library without a GPU: it loads, exports every function include/*.h declares,
and rejects bad arguments the way the reference does (fatal "raceline: fatal: ..." and exit
status 1 by default, src/metal_rt.mm:16-24), before any device work."""

import glob
import os
import re
import subprocess
import sys

import pytest

from raceline_amd import lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names += re.findall(r"\b((?:rlq|rlm|rl)_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_path():
    names = declared_functions()
    for must in ("rlq_linear_affine", "rlq_dequant_affine", "rlq_repack_blocked", "rlq_group_sums",
                 "rlq_pack_affine", "rlq_pack_affine_blocked", "rlq_packed_affine_bytes"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = lib.load()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    # the ctypes binding declares every one of them
    assert set(declared_functions()) <= set(lib.SIGNATURES)
    nm = subprocess.run(["nm", "-D", "--defined-only", lib.library_path()], capture_output=True, text=True)
    if nm.returncode == 0:
        exported = set(re.findall(r"\b((?:rlq|rlm|rl)_\w+)\b", nm.stdout))
        assert set(declared_functions()) <= exported


def test_abi_version_and_workspace_query():
    L = lib.load()
    assert L.rlq_abi_version() == 1
    assert L.rlq_linear_workspace_bytes(64, 4096, 4096) > 0     # the prefill kernel stages group sums
    assert L.rlq_linear_workspace_bytes(1, 100, 4096) == 0      # invalid K: nothing to size
    # packed layout: 2304 bytes per (16-row tile, quad of groups of 64)
    assert L.rlq_packed_affine_bytes(4096, 4096) == 256 * 16 * 2304
    assert L.rlq_packed_affine_bytes(64, 33) == 3 * 1 * 2304
    assert L.rlq_linear_workspace_bytes(256, 4096, 1024) > L.rlq_linear_workspace_bytes(64, 4096, 1024)
    # the decode kernel splits K for few tiles and a long K (27B down: 7 splits): 4096 bytes
    # of counters, then 7 x M x N partial floats; a workspace sized for M serves smaller M
    assert L.rlq_linear_workspace_bytes(8, 17408, 5120) >= 4096 + 7 * 8 * 5120 * 4
    assert L.rlq_linear_workspace_bytes(1, 17408, 5120) >= 4096 + 7 * 1 * 5120 * 4
    assert L.rlq_linear_workspace_bytes(64, 17408, 5120) >= L.rlq_linear_workspace_bytes(8, 17408, 5120)


def test_split_decode_without_workspace_is_an_error():
    """A decode call on a weight whose K the kernel splits (here 7 ways: K = 17408, N = 640)
    needs the workspace for its partial sums and counters: without it the call fails before
    any launch (pointers are placeholders, never dereferenced)."""
    with pytest.raises(lib.RlqError, match="splits K in 7"):
        lib.call("rlq_linear_affine", 16, 17408, 1, 17408, 640, 16, 0, 16, 640, 0, None, 0, None)


def test_bad_arguments_return_an_error_in_nonfatal_mode():
    with pytest.raises(lib.RlqError, match="multiple of the group size"):
        lib.call("rlq_linear_affine", 16, 100, 1, 100, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="unknown scale dtype"):
        lib.call("rlq_linear_affine", 16, 64, 1, 64, 10, 16, 7, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="x_stride"):
        lib.call("rlq_linear_affine", 16, 60, 1, 64, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="null pointer"):
        lib.call("rlq_linear_affine", None, 64, 1, 64, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="16-byte aligned"):
        lib.call("rlq_linear_affine", 8, 64, 1, 64, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="unknown kernel"):
        lib.call("rlq_linear_affine_kernel", 5, 16, 64, 1, 64, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="decode kernel handles M <= 8"):
        lib.call("rlq_linear_affine_kernel", 1, 16, 64, 9, 64, 10, 16, 0, 16, 10, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="workspace"):
        lib.call("rlq_linear_affine_kernel", 2, 16, 4096, 64, 4096, 1024, 16, 0, 16, 1024, 0, None, 0, None)
    with pytest.raises(lib.RlqError, match="block 256"):
        lib.call("rlq_pack_affine_blocked", 16, 16, 16, 64, 300, 0, 10, 16, None)
    with pytest.raises(lib.RlqError, match="block 256"):
        lib.call("rlq_repack_blocked", 16, 16, 16, 64, 300, 0, 10, 16, 16, 16, None)
    with pytest.raises(lib.RlqError, match="outside"):
        lib.call("rlq_repack_blocked", 16, 16, 16, 64, 256, 200, 100, 16, 16, 16, None)
    assert lib.load().rlq_last_error().decode().startswith("rlq_repack_blocked")


def test_errors_are_fatal_by_default():
    code = ("import ctypes, sys; sys.path.insert(0, %r); from raceline_amd import lib; "
            "L = ctypes.CDLL(lib.library_path()); "
            "L.rlq_linear_affine(ctypes.c_void_p(16), 100, 1, 100, 10, ctypes.c_void_p(16), 0, "
            "ctypes.c_void_p(16), 10, 0, None, ctypes.c_size_t(0), None); "
            "print('not reached')") % ROOT
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
    assert "raceline: fatal: rlq_linear_affine: K=100 is not a multiple of the group size 64" in r.stderr
    assert "not reached" not in r.stdout


def test_no_alloc_moe_refuses_sizes_past_its_scratch():
    """rlq_moe_no_alloc holds a fixed scratch array; a call that needs more is refused with an
    error naming the limit, before any device work."""
    L = lib.load()
    cap = L.rlq_moe_no_alloc_max_bytes()
    assert cap == 48 << 20
    assert L.rlq_moe_workspace_bytes(512, 256, 8, 2048, 512) <= cap
    assert L.rlq_moe_workspace_bytes(4096, 256, 8, 2048, 512) > cap
    with pytest.raises(lib.RlqError, match="more than the 50331648 it holds"):
        lib.call("rlq_moe_no_alloc", 16, 2048, 16, 257, 4096, 256, 8, 1, 2048, 512, 16, 16, 0, 16, 2048, None)


def test_raw_native_product_refuses_the_half_step_book():
    with pytest.raises(lib.RlqError, match="no half step"):
        lib.call("rlq_linear_native_raw", 16, 64, 1, 64, 16, 16, 2, 16, 16, None, 0, None)
