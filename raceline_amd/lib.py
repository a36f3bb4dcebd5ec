"""ctypes binding of libraceline_amd.so (the C ABI of include/rlq.h).

Discovery follows raceline/engine.py:67-81 of the reference: the library named by
RACELINE_LIB if set, else the one built next to this package. There is no fallback:
without the built library every call raises, so nothing silently runs on the CPU.
The binding puts the library in non-fatal mode and turns a failed call into a
RuntimeError carrying the library's message.
"""

from __future__ import annotations

import ctypes
import functools
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libraceline_amd.so"

c_int, c_size_t, c_void_p, c_char_p = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p

# name -> (restype, argtypes); the whole exported surface of include/rlq.h
SIGNATURES = {
    "rlq_abi_version": (c_int, []),
    "rlq_set_fatal": (c_int, [c_int]),
    "rlq_last_error": (c_char_p, []),
    "rlq_set_device": (c_int, [c_int]),
    "rlq_packed_affine_bytes": (c_size_t, [c_int, c_int]),
    "rlq_pack_affine": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "rlq_pack_affine_blocked": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                        c_void_p]),
    "rlq_repack_blocked": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                   c_void_p, c_void_p]),
    "rlq_linear_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "rlq_linear_affine": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_int, c_int,
                                  c_void_p, c_size_t, c_void_p]),
    "rlq_linear_affine_kernel": (c_int, [c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p,
                                         c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "rlq_group_sums": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rlq_dequant_affine": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rlq_stream_read": (c_int, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "rlq_packed_codes_bytes": (c_size_t, [c_int, c_int]),
    "rlq_pack_codes": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "rlq_pack_native_blocked": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rlq_linear_native": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int,
                                  c_int, c_void_p, c_size_t, c_void_p]),
    "rlq_linear_native_kernel": (c_int, [c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int,
                                         c_void_p, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "rlq_linear_native_raw": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_int,
                                      c_void_p, c_size_t, c_void_p]),
    "rlq_packed_f16_bytes": (c_size_t, [c_int, c_int]),
    "rlq_pack_f16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "rlq_pack_f16_blocked": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rlq_linear_f16": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "rlq_pack_moe_gate_up": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "rlq_moe_max_items": (c_size_t, [c_int, c_int, c_int]),
    "rlq_moe_route": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_void_p]),
    "rlq_moe_gate_up": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "rlq_moe_down": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p,
                             c_void_p, c_int, c_void_p]),
    "rlq_moe_combine": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "rlq_moe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "rlq_moe_linear_native": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                      c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p]),
    "rlq_moe_swiglu": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "rlq_moe_native": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_int,
                               c_void_p, c_size_t, c_void_p]),
    "rlq_moe_gate_up_native": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                       c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "rlq_moe": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p,
                        c_void_p, c_int, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    # include/rl_engine.h: the model file reader and the engine layer
    "rlm_open": (c_void_p, [c_char_p]),
    "rlm_close": (None, [c_void_p]),
    "rlm_config_int": (c_int, [c_void_p, c_char_p]),
    "rlm_tensor": (c_int, [c_void_p, c_char_p, c_void_p]),
    "rlm_tensor_part": (c_int, [c_void_p, c_char_p, c_char_p, c_void_p, c_void_p]),
    "rlm_section": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "rl_open": (c_void_p, [c_char_p, c_int, c_int]),
    "rl_close": (None, [c_void_p]),
    "rl_vocab": (c_int, [c_void_p]),
    "rl_hidden_size": (c_int, [c_void_p]),
    "rl_linear": (c_int, [c_void_p, c_char_p, c_char_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p]),
    "rl_norm": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p]),
    "rl_mlp": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_void_p]),
    "rl_head": (c_void_p, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "rl_set_draft_vocab": (None, [c_void_p, c_int]),
    "rl_set_draft_tail": (None, [c_void_p, c_int]),
    "rl_draft_main": (c_int, [c_void_p]),
    "rl_draft_tail": (c_int, [c_void_p]),
    "rl_draft_vocab": (c_int, [c_void_p]),
    "rl_logits_stride": (c_size_t, [c_void_p]),
    "rl_expert_cache": (c_int, [c_void_p, c_void_p, c_void_p]),
    "rl_expert_cache_size": (None, [c_void_p, c_void_p, c_void_p]),
    "rl_draft_head": (c_void_p, [c_void_p, c_void_p, c_void_p]),
    "rl_top_k": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "rl_top_k_device": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "rl_argmax": (c_int, [c_void_p]),
    "rlq_moe_no_alloc_max_bytes": (c_size_t, []),
    "rlq_moe_no_alloc": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                 c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p]),
}


def library_path() -> str:
    env = os.environ.get("RACELINE_LIB")
    for path in (env, os.path.join(HERE, LIB_NAME)):
        if path and os.path.isfile(path):
            return path
    raise RuntimeError(f"{LIB_NAME} not found: build it with `python -m raceline_amd.build` "
                       "(or __graft_entry__.build()) or point RACELINE_LIB at it")


@functools.lru_cache(maxsize=1)
def load() -> ctypes.CDLL:
    lib = ctypes.CDLL(library_path())
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


class RlqError(RuntimeError):
    pass


def call(name: str, *args):
    """Calls rlq_<name> in non-fatal mode and raises RlqError on a nonzero status."""
    lib = load()
    lib.rlq_set_fatal(0)
    rc = getattr(lib, name)(*args)
    if isinstance(rc, int) and rc != 0 and SIGNATURES[name][0] is c_int and name not in (
            "rlq_abi_version", "rlq_set_fatal"):
        raise RlqError(f"{name}: {lib.rlq_last_error().decode(errors='replace')}")
    return rc
