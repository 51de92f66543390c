"""ctypes binding of libqlora_amd.so (the C-ABI declared in include/qlora_amd.h).

The library is loaded from this package's directory (built in-tree by build.py). There is no
fallback: if it is missing or fails to load, every op raises. A non-zero return code of an entry
point becomes a RuntimeError naming the entry point and the HIP error.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqlora_amd.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float

# entry point -> argument types (in the order of include/qlora_amd.h); all return int
SIGNATURES = {
    "qlora_nf4_dequant": [P, P, P, P, P, P, P, I64, I32, I32, I32, I32, I64, I64, P],
    "qlora_nf4_dequant_many": [I32, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P],
    "qlora_nf4_dequant_many_timed": [I32, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P],
    "qlora_dropout_keep": [P, I64, I64, I64, I64, F32, I32, P],
    "qlora_dropout_keep_below": [F32, P],
    "qlora_rms_fwd": [P, P, P, I32, P, P, P, P, P, P, I64, I64, F32, F32, F32, I64, I64, I64,
                      I64, I32, I32, I32, I32, I32, P, P, P, P],
    "qlora_rms_bwd": [P, P, P, P, P, P, I32, P, P, P, P, I64, I64, I64, F32, F32, I64, I64,
                      I64, I64, F32, I32, I32, I32, I32, P, P, P, F32, P, I32, P],
    "qlora_rope_fwd": [P, P, P, P, P, I64, P, P, P, P, I64, I32, I32, I32, I32, F32, P],
    "qlora_rope_bwd": [P, P, P, P, P, I64, P, P, I64, I32, I32, I32, I32, P],
    "qlora_glu_fwd": [P, P, I64, I64, P],
    "qlora_glu_bwd": [P, P, I64, I64, P],
    "qlora_ce": [P, I64, P, P, P, P, I64, I64, I32, P],
    "qlora_ce_piece": [P, I64, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, P],
    "qlora_ce_finish": [P, P, P, P, P, P, P, P, P, P, I64, I64, I64, P],
    "qlora_ce_grad": [P, I64, P, P, I64, I64, I64, P],
    "qlora_nf4_block_scales": [P, P, P, P, I32, I32, I64, I64, I64, P, P],
    "qlora_nf4_gemm": [P, I64, P, P, P, I32, I32, I64, I64, P, I64, P, P, I64, I64, I32, I32,
                       I64, I32, P, I64, P],
    "qlora_gemm16": [P, I64, P, I64, I64, I64, I64, I32, P, I64, P, P, I64, I32, I64, P, I64,
                     I32, I32, I32, P, I64, P],
    "qlora_gemm16_timed": [P, I64, P, I64, I64, I64, I64, I32, P, I64, P, P, I64, I32, I64, P,
                           I64, I32, I32, I32, P, I64, P, P, P],
    "qlora_gemm16_f32": [P, I64, P, I64, I64, I64, I64, I32, P, I64, F32, P, P, I64, I32, I32,
                         I32, P, I64, P],
    "qlora_gemm16_workspace": [I64, I64, I64, I32, I32, I32, I32, I32, P],
    "qlora_gemm16_plan": [I64, I64, I64, I32, I32, P, P, P],
    "qlora_gemm16_parts": [P, I64, P, I64, I64, I64, I64, I32, I32, I32, I32, P, I64, P],
    "qlora_gemm16_plan_split": [I64, I64, I64, I32, I32, P, P, P, P, P],
    "qlora_resid_add": [P, P, P, I64, P],
    "qlora_lora_fwd_rows": [P, P, P, P, P, P, P, P, P, P, I64, I32, I32, I32, I32, P],
    "qlora_lora_bwd_rows": [P, P, I64, P, P, P, P, P, P, P, P, I64, I32, I32, I32, I32, F32, P],
    "qlora_lora_grad_workspace": [I64, I32, I32, I32, I32, P],
    "qlora_lora_grad": [P, P, I64, P, P, P, P, P, P, P, P, P, P, I64, I32, I32, I32, I32, F32, P,
                        I64, P],
    "qlora_lora_grad_noalloc": [P, P, I64, P, P, P, P, P, P, P, P, P, P, I64, I32, I32, I32, I32,
                                F32, P],
    "qlora_nf4_quantize": [P, I32, I64, P, P, P],
    "qlora_nf4_quantize_stats_workspace": [I64, P],
    "qlora_nf4_quantize_stats": [P, I64, P, P, I64, P, P, P, P],
    "qlora_attn_fwd": [P, P, P, P, P, P, I32, I32, I64, I32, I32, I32, F32, P],
    "qlora_attn_bwd": [P, P, P, P, P, P, P, P, P, P, P, I32, I32, I64, I32, I32, I32, F32, P],
    "qlora_attn_split_workspace": [I32, I64, I32, I32, I32, P],
    "qlora_attn_fwd_split": [P, P, P, P, P, P, I32, I32, I64, I32, I32, I32, F32, I32, P, I64, P],
    "qlora_attn_bwd_split": [P, P, P, P, P, P, P, P, P, P, P, I32, I32, I64, I32, I32, I32, F32,
                             I32, P, I64, P],
}

_lib = None
HOOKS = {}  # entry point -> object with .call(fn, args) (profiling.LaunchTimer)


class LibraryMissing(RuntimeError):
    pass


def load():
    """The loaded library (ctypes.CDLL), loading and binding it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950) first")
    lib = ctypes.CDLL(LIB_PATH)
    lib.qlora_error_string.restype = ctypes.c_char_p
    lib.qlora_error_string.argtypes = [ctypes.c_int]
    lib.qlora_abi_version.restype = ctypes.c_int
    lib.qlora_abi_version.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    _lib = lib
    return lib


_FNS = {}


def call(name, *args):
    """Call entry point `name`; raise RuntimeError on a non-zero return code."""
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    hook = HOOKS.get(name) if HOOKS else None
    rc = hook.call(fn, args) if hook is not None else fn(*args)
    if rc != 0:
        msg = load().qlora_error_string(rc).decode(errors="replace")
        raise RuntimeError(f"{name} failed: hipError {rc} ({msg})")
    return rc


def exported_symbols():
    """Names of the qlora_* entry points the built library exports (reads the ELF dynamic
    symbol table through the loader; no device call)."""
    lib = load()
    found = []
    for name in list(SIGNATURES) + ["qlora_error_string", "qlora_abi_version"]:
        try:
            getattr(lib, name)
            found.append(name)
        except AttributeError:
            pass
    return found
