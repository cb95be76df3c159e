"""ctypes binding of libress_hip.so (the C ABI declared in include/ress_hip.h).

The library is built in-tree by `ress_amd.build` (or `__graft_entry__.build()`).
There is no fallback: if the library is missing, or the device is not a GPU, every
call raises.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libress_hip.so")

# argument codes: p = pointer, i = int, l = long long, f = float, d = double, s = stream
_SIGS = {
    "ress_prep_qkv": "pppiiiii" + "p" + "lllllllll" + "ppppppppppppp" + "i" + "s",
    "ress_per_block_int8": "pppiiii" + "llllll" + "ppppp" + "s",
    "ress_prep_kv_plain": "ppiii" + "llllll" + "ppppp" + "s",
    "ress_pooled_scores": "ppiiiifpp" + "s",
    "ress_baseline_budget": "plifip" + "s",
    "ress_head_budget": "piiipdiiipp" + "s",
    "ress_select_blocks": "ppiiiiiiippp" + "s",
    "ress_fill_block_map": "ppplI" + "s",
    "ress_block_map_lut": "plipp" + "s",
    "ress_sparse_attn_fwd": "pppppppippiiiii" + "p" + "fpilllps",
    "ress_sparse_attn_fwd_f16": "plllppppp" + "iiiii" + "pf" + "pi" + "lll" + "ps",
    "ress_sparse_attn_fwd_f16_noalloc": "plllppppp" + "iiiii" + "pf" + "pi" + "lll" + "s",
    "ress_qattn_block_sparse_fwd": "pppipipppppiiiilllllliiifipls",
    "ress_restore_swap": "pppp" + "iiiiii" + "dd" + "i" + "ppp" + "pl" + "s",
    "ress_meansim_block_map": "ppp" + "iiii" + "llllll" + "ppi" + "ppppppppp" + "pl" + "s",
    "ress_qk_norm_rope": "piii" + "pppp" + "f" + "pf" + "ppp" + "s",
    "ress_bf16_selfcheck": "Il" + "p" + "s",
}
_CT = {
    "p": ctypes.c_void_p,
    "i": ctypes.c_int,
    "I": ctypes.c_int,
    "l": ctypes.c_longlong,
    "f": ctypes.c_float,
    "d": ctypes.c_double,
    "s": ctypes.c_void_p,
}

_lib = None


def lib():
    """The loaded library (loads on first use; raises if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ress_amd.build` "
                "(the HIP kernels are the only implementation; there is no fallback)")
        L = ctypes.CDLL(LIB_PATH)
        L.ress_last_error.restype = ctypes.c_char_p
        L.ress_abi_version.restype = ctypes.c_int
        L.ress_qattn_workspace_size.restype = ctypes.c_longlong
        L.ress_qattn_workspace_size.argtypes = [ctypes.c_int] * 4
        L.ress_attn_sched_bytes.restype = ctypes.c_longlong
        L.ress_attn_sched_bytes.argtypes = [ctypes.c_int] * 3
        L.ress_restore_swap_workspace_size.restype = ctypes.c_longlong
        L.ress_restore_swap_workspace_size.argtypes = [ctypes.c_int] * 4
        L.ress_meansim_workspace_size.restype = ctypes.c_longlong
        L.ress_meansim_workspace_size.argtypes = [ctypes.c_int] * 4
        L.ress_noalloc_scratch_bytes.restype = ctypes.c_longlong
        L.ress_noalloc_scratch_bytes.argtypes = []
        L.ress_noalloc_status_address.restype = ctypes.c_int
        L.ress_noalloc_status_address.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        for name, sig in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [_CT[c] for c in sig]
        _lib = L
    return _lib


def ptr(t):
    """Device pointer of a tensor (None -> NULL). Refuses CPU tensors."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError("libress_hip kernels take device tensors; got a CPU tensor")
    return t.data_ptr()


def stream_handle(device=None):
    return torch.cuda.current_stream(device).cuda_stream


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().ress_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def last_error():
    return lib().ress_last_error().decode(errors="replace")


def exported_symbols():
    return list(_SIGS) + ["ress_last_error", "ress_abi_version", "ress_qattn_workspace_size",
                          "ress_attn_sched_bytes", "ress_restore_swap_workspace_size", "ress_meansim_workspace_size",
                          "ress_noalloc_scratch_bytes",
                          "ress_noalloc_status_address"]
