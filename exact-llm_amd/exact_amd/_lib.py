"""ctypes binding of libexact_hip.so (the C ABI declared in include/exact_hip.h).

The library is the only compute path: if it is missing or fails to load this module raises,
there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libexact_hip.so")

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
U64 = ctypes.c_uint64

# name -> argument types (all return int status except where noted)
SIGNATURES = {
    "exact_synth_linear": [U64, U64, I32, I32, P, P, P, I32, I32, I32, I32, P],
    "exact_synth_vector": [U64, I64, I64, P, I64, P],
    "exact_pack_linear": [P, P, P, P, I32, I32, I32, I32, P],
    "exact_pack_scales": [P, P, I32, I32, I32, I32, P],
    "exact_gemv": [P, P, P, P, I32, I32, P],
    "exact_gemv_g128": [P, I32, P, P, P, P, I32, I32, I32, P],
    "exact_gemv_g128_acc": [P, I32, P, P, P, P, I32, I32, I32, P],
    "exact_gemm_g128": [P, I32, P, P, P, P, I32, I32, I32, P],
    "exact_gemm_g128_zeroed": [P, I32, P, P, P, P, I32, I32, I32, P],
    "exact_gemm_g128_a16": [P, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_gemm_g128_a16_zeroed": [P, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_gemm_g128_digits": [P, P, P, P, P, P, I32, I32, I32, I32, P],
    "exact_gemv_g128_qrow_acc": [P, I64, P, I32, I32, P, P, P, P, P, I32, I32, I32, P, I64, P],
    "exact_gemv_g128_swiglu": [P, P, P, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_gemv_g128_norm_acc": [P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_gemv_g128_norm_acc_blockwaves": [I32, I32, I32, I32],
    "exact_gemv_g128_norm_swiglu": [P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_requant_group": [P, P, P, P, I32, I32, P],
    "exact_requant_channel": [P, P, P, I32, P, P, I32, I32, P],
    "exact_qrow": [P, I32, P, P, I32, I32, P],
    "exact_irms": [P, P, P, I32, I32, P],
    "exact_rmsnorm_qrow": [P, P, P, P, I32, P, P, I32, I32, I32, P, P],
    "exact_swiglu_qrow": [P, P, P, I32, P, P, P, I32, I32, I32, P, P, P],
    "exact_quant_rows": [P, I64, P, I32, I32, P, P, I32, I32, I32, P, P, I64, P],
    "exact_isilu": [P, P, P, I64, P],
    "exact_isig": [P, P, P, I64, P],
    "exact_isoftmax": [P, P, P, P, I32, I32, P],
    "exact_qkv_rope_cache": [P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, P],
    "exact_attention": [P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, P],
    "exact_attention_qkv": [P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, P],
    "exact_attention_qkv_split": [P, P, P, P, P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, I32, P],
    "exact_attention_prefill": [P, P, P, P, P, I32, P, P, P, P, P, I64, I32, I32, I32, I32, I32, I32, I32, P],
    "exact_embed": [P, P, P, I32, I32, I32, P],
    "exact_embed_table": [P, P, P, I32, I32, P],
    "exact_logits_argmax": [P, P, P, P, P, I32, I32, I32, P],
    "exact_logits_argmax_noalloc": [P, P, P, P, I32, I32, I32, P],
    "exact_advance": [P, I32, P],
    "exact_zero": [P, I64, P],
    "exact_sample": [P, I32, I32, U64, P, I64, P, P, P, P],
    "exact_router_topk": [P, I32, P, P, P, P, I32, P, P, I32, I32, I32, I32, P],
    "exact_moe_dispatch": [P, P, P, P, P, P, P, P, P, I32, I32, I32, I32, P],
    "exact_moe_route": [P, I32, P, P, P, P, I32, P, P, I32, I32, I32, I32, P, P, P, P, P, P, P, I32, P],
    "exact_gemv_g128_experts": [P, I32, P, P, P, I64, I64, P, P, P, P, I32, P, I32, I32, P],
    "exact_gemm_g128_experts": [P, I32, P, P, P, I64, I64, P, P, P, P, P, P, I32, P, I32, I32, I32, P],
    "exact_gemv_g128_experts_swiglu": [P, P, P, P, I64, I64, P, P, P, P, I32, I32, P, P, P, P, I32, I32, P],
    "exact_gemv_g128_experts_qrow_acc": [P, I64, P, I32, P, P, I64, I64, P, P, P, P, I32, I32, P, P, I32, I32, P],
    "exact_moe_swiglu_pair": [P, P, P, P, I64, I64, P, P, P, P, I32, I32, P, P, P, P, I32, P, P, P, P, P, P, I32, I32, I32, P],
    "exact_moe_qrow_pair": [P, I64, P, I32, P, P, I64, I64, P, P, P, P, I32, I32, P, P, I32, I32, P, I64, P, I32, P, P, P, P, P,
                            I32, I32, I32, P, I64, P],
    "exact_moe_combine": [P, P, P, P, P, P, P, P, I32, I32, I32, I32, P],
}
OTHER = {"exact_version": ([], ctypes.c_int), "exact_last_error": ([], ctypes.c_char_p),
         "exact_attention_prefill_workspace": ([I32, I32, I32, I32, I32], ctypes.c_int64)}
ERRORS = {1: "bad argument", 2: "unsupported size", 3: "HIP launch error"}


class ExactError(RuntimeError):
    pass


_LIB = None


def load():
    """Load the library (importing torch first so the library binds to torch's HIP runtime)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ExactError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C exact-llm_amd)")
    import torch  # noqa: F401  (one HIP runtime per process: torch's)
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = ctypes.c_int
    for name, (args, res) in OTHER.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    _LIB = lib
    return lib


def call(name, *args):
    rc = getattr(load(), name)(*args)
    if rc != 0:
        msg = ERRORS.get(rc, "error")
        detail = load().exact_last_error().decode() if rc == 3 else ""
        raise ExactError(f"{name}: {msg} (code {rc}) {detail}".strip())
