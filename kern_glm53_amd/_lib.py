"""ctypes binding of libkg.so (the C ABI declared in include/kg.h).

The library is loaded from this package directory.  It must have been built (`kern_glm53_amd.build`);
there is no fallback path: a missing library raises at first use.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libkg.so"

P = ctypes.c_void_p
I = ctypes.c_int
LL = ctypes.c_longlong

# name -> argtypes (the trailing void* is the hipStream_t)
SIGNATURES = {
    "kg_fp8_gemm": [P, P, P, P, P, I, I, I, I, I, I, I, P],
    "kg_fp8_gemm_psum": [P, P, P, P, P, P, I, I, I, I, I, I, I, P],
    "kg_fp8_gemm_psum_silu_quant": [P, P, P, P, P, I, I, I, I, I, I, P, P, I, P],
    "kg_fp8_weight_frag": [P, P, LL, I, P],
    "kg_fp8_gemm_wf": [P, P, P, P, P, I, I, I, I, I, I, I, P],
    "kg_fp8_gemm_psum_wf": [P, P, P, P, P, P, I, I, I, I, I, I, I, P],
    "kg_fp8_gemm_psum_silu_quant_wf": [P, P, P, P, P, I, I, I, I, I, I, P, P, I, P],
    "kg_bf16_batched": [P, P, P, I, I, I, I, I, LL, LL, LL, LL, LL, LL, P],
    "kg_mqa_logits": [P, P, P, P, P, P, P, I, I, I, P],
    "kg_gemm_bf16": [P, P, P, I, I, I, I, P],
    "kg_gemm_bf16_f32": [P, P, P, I, I, I, I, P],
    "kg_quant": [P, I, P, P, I, I, I, P],
    "kg_silu_mul_quant": [P, I, P, P, I, P, I, P],
    "kg_moe_routing": [P, I, I, I, I, P, P, P, P, P, P, P, P],
    "kg_moe_psum": [P, P, P],
    "kg_moe_gather": [P, P, I, P, P, P, I, I, P],
    "kg_moe_combine": [P, P, P, P, P, I, P],
    "kg_router_topk": [P, P, P, P, P, I, P],
    "kg_requant": [P, P, P, P, I, I, I, I, I, I, LL, P],
    "kg_kvb": [P, P, P, P, P],
    "kg_add_rms_quant": [P, P, P, P, P, P, I, I, P],
    "kg_mla_prep": [P, I, P, P, P, P, P, P, P, P, P, P, P, I, I, LL, I, P],
    "kg_mla_prep_fp8": [P, I, P, P, P, P, P, P, P, P, P, P, P, I, I, LL, I, P],
    "kg_q_post": [P, I, P, P, P, P, P, P, I, I, I, P],
    "kg_topk_prefill": [P, P, P, P, I, I, I, I, I, P],
    "kg_topk_stream": [P, P, P, P, I, P],
    "kg_topk_slots": [P, P, I, P, P, P, I, P],
    "kg_idx_gather": [P, P, I, P, I, P, P, I, P],
    "kg_kv_dequant": [P, P, I, P, I, P, I, P],
}

_lib = None
_lock = threading.Lock()


class KgError(RuntimeError):
    """A libkg entry point returned a non-zero hipError_t."""

    def __init__(self, name: str, code: int):
        what = "invalid argument (host-side validation)" if code == 1 else f"hipError_t {code}"
        super().__init__(f"{name}: {what}")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(f"{LIB_PATH} is not built: run `python -m kern_glm53_amd.build` "
                                       "(there is no CPU fallback for these kernels)")
                l = ctypes.CDLL(str(LIB_PATH))
                for name, argtypes in SIGNATURES.items():
                    f = getattr(l, name)
                    f.argtypes = argtypes
                    f.restype = ctypes.c_int
                l.kg_version.argtypes = []
                l.kg_version.restype = ctypes.c_char_p
                _lib = l
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise KgError(name, rc)
