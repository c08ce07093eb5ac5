"""ctypes binding of libfa_rocm.so (include/fa_rocm.h) and libfa_synth.so.

The HIP library is required: importing the compute entry points without it
raises, there is no CPU fallback.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import re
import weakref

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "_lib")
ROOT = os.path.dirname(_HERE)
HEADER = os.path.join(ROOT, "include", "fa_rocm.h")
SYNTH_HEADER = os.path.join(ROOT, "include", "fa_synth.h")

FA_OK, FA_ERR_ARG, FA_ERR_HIP, FA_ERR_OOM, FA_ERR_STATE, FA_ERR_UNSUPPORTED = range(6)
FA_DT_F32, FA_DT_BF16 = 0, 1
FA_ACT_NONE, FA_ACT_RELU, FA_ACT_GELU, FA_ACT_TANH = 0, 1, 2, 3
FA_B_KN, FA_B_NK = 0, 1
KERNEL_KINDS = ["gemm_qkv", "gemm_o", "gemm_gateup", "gemm_down", "gemm_head", "attention", "qknorm_rope",
                "residual_norm", "gather", "pool_l2", "gemm_ple", "ple_norm"]

i32, i64, f32, f64, vp = C.c_int32, C.c_int64, C.c_float, C.c_double, C.c_void_p
P_f32 = C.POINTER(C.c_float)
P_i32 = C.POINTER(C.c_int32)
P_i64 = C.POINTER(C.c_int64)


class FaError(RuntimeError):
    """Error status from the C ABI: code (FA_ERR_*) and the library's message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.msg = msg


class Epilogue(C.Structure):
    _fields_ = [("bias", vp), ("row_scale", vp), ("act", C.c_int), ("mul", vp), ("ldm", i64),
                ("residual", vp), ("ldr", i64)]


FA_MAX_BATCH_DIMS = 8


class Matrix(C.Structure):
    """fa_matrix: a strided operand (data, row/column strides, batch strides; elements)."""
    _fields_ = [("data", vp), ("rs", i64), ("cs", i64), ("bstride", i64 * FA_MAX_BATCH_DIMS)]


class GemmaConfig(C.Structure):
    _fields_ = [("hidden_size", i32), ("num_hidden_layers", i32), ("num_attention_heads", i32),
                ("num_key_value_heads", i32), ("head_dim", i32), ("intermediate_size", i32), ("vocab_size", i32),
                ("sliding_window", i32), ("use_bidirectional", i32), ("sliding_window_pattern", i32),
                ("rope_local_base_freq", f64), ("rope_theta", f64), ("query_pre_attn_scalar", f64),
                ("rms_norm_eps", f32), ("max_tokens", i32), ("n_dense", i32), ("dense_out", i32 * 4),
                ("variant", i32), ("hidden_size_per_layer_input", i32), ("embedding_dim", i32),
                ("layer_head_dim", i32 * 64), ("layer_kv_heads", i32 * 64), ("layer_sliding", i32 * 64),
                ("dense_act", i32 * 4)]


_SIGS = {
    "fa_create": (C.c_int, [C.c_int, C.POINTER(vp)]),
    "fa_destroy": (None, [vp]),
    "fa_last_error": (C.c_char_p, [vp]),
    "fa_stream": (vp, [vp]),
    "fa_sync": (C.c_int, [vp]),
    "fa_version": (C.c_char_p, []),
    "fa_device_alloc": (C.c_int, [vp, C.c_size_t, C.POINTER(vp)]),
    "fa_device_free": (C.c_int, [vp, vp]),
    "fa_memcpy_h2d": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "fa_memcpy_d2h": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "fa_matmul_fused": (C.c_int, [vp, i64, i64, i64, vp, i64, vp, i64, C.c_int, C.c_int, C.POINTER(Epilogue), vp,
                                  i64]),
    "fa_matmul_fused_dev": (C.c_int, [vp, i64, i64, i64, vp, i64, vp, i64, C.c_int, C.c_int, C.POINTER(Epilogue),
                                      vp, i64]),
    "fa_matmul_strided": (C.c_int, [vp, i32, P_i64, i64, i64, i64, C.POINTER(Matrix), C.POINTER(Matrix),
                                    C.POINTER(Epilogue), vp]),
    "fa_matmul_strided_dev": (C.c_int, [vp, i32, P_i64, i64, i64, i64, C.POINTER(Matrix), C.POINTER(Matrix),
                                        C.POINTER(Epilogue), vp]),
    "fa_row_sum_squares": (C.c_int, [vp, vp, i64, i64, vp]),
    "fa_rmsnorm": (C.c_int, [vp, vp, vp, f32, i64, i64, vp]),
    "fa_rope": (C.c_int, [vp, vp, f64, vp, i64, i32, i32, vp]),
    "fa_attention": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, vp, i64, i64,
                               i64, i64, f32, vp]),
    "fa_attention_dev": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, vp, i64,
                                   i64, i64, i64, f32, vp]),
    "fa_similarities_topk": (C.c_int, [vp, vp, i64, vp, i64, i32, i32, vp, vp]),
    "fa_similarities_topk_dev": (C.c_int, [vp, vp, i64, vp, i64, i32, i32, vp, vp]),
    "fa_similarities_topk_dev_noalloc": (C.c_int, [vp, vp, i64, vp, i64, i32, i32, vp, vp]),
    "fa_cluster_normalize": (C.c_int, [vp, vp, i64, i32, vp]),
    "fa_cluster_normalize_dev": (C.c_int, [vp, vp, i64, i32, vp]),
    "fa_cluster_nearest": (C.c_int, [vp, vp, i64, vp, i64, i32, vp, vp]),
    "fa_cluster_nearest_dev": (C.c_int, [vp, vp, i64, vp, i64, i32, vp, vp]),
    "fa_cluster_kmeans": (C.c_int, [vp, vp, i64, i32, i32, i32, C.c_uint64, vp, vp, vp, vp, C.POINTER(i32)]),
    "fa_cluster_kmeans_dev": (C.c_int, [vp, vp, i64, i32, i32, i32, C.c_uint64, vp, vp, vp, vp, C.POINTER(i32)]),
    "fa_gemma_create": (C.c_int, [vp, C.POINTER(GemmaConfig), C.POINTER(vp)]),
    "fa_gemma_destroy": (None, [vp]),
    "fa_gemma_set_weight": (C.c_int, [vp, C.c_char_p, C.c_int, P_i64, i32, vp]),
    "fa_gemma_finalize": (C.c_int, [vp]),
    "fa_gemma_embed_ids": (C.c_int, [vp, vp, vp, i32, i32, i32, vp]),
    "fa_gemma_embed_ids_dev": (C.c_int, [vp, vp, vp, i32, i32, i32, vp]),
    "fa_gemma_encode_ids": (C.c_int, [vp, vp, vp, i32, i32, i32, vp]),
    "fa_gemma_encode_ids_dev": (C.c_int, [vp, vp, vp, i32, i32, i32, vp]),
    "fa_gemma_set_profiling": (C.c_int, [vp, C.c_int]),
    "fa_gemma_kernel_stats": (C.c_int, [vp, C.c_int, P_i64, C.POINTER(f64), C.POINTER(f64), C.POINTER(f64)]),
    "fa_gemma_reset_stats": (C.c_int, [vp]),
}

_SYNTH_SIGS = {
    "fa_synth_normal_bf16": (None, [C.c_uint64, C.c_char_p, f64, i64, vp]),
    "fa_synth_normal_f32": (None, [C.c_uint64, C.c_char_p, f64, i64, vp]),
    "fa_bf16_to_f32": (None, [vp, i64, vp]),
    "fa_f32_to_bf16": (None, [vp, i64, vp]),
    "fa_synth_uniform_i32": (None, [C.c_uint64, C.c_char_p, i32, i32, i64, vp]),
    "fa_synth_zipf_i32": (C.c_int, [C.c_uint64, C.c_char_p, f64, i32, i32, i64, vp]),
    "fa_synth_unit_rows": (None, [C.c_uint64, C.c_char_p, i64, i32, vp]),
}

_lib = None
_synth = None


def lib_path() -> str:
    return os.path.join(LIB_DIR, "libfa_rocm.so")


def lib() -> C.CDLL:
    """The HIP library; raises if it was not built."""
    global _lib
    if _lib is None:
        p = lib_path()
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is missing: build it with `python -m ai_amd.build` (no CPU fallback exists)")
        l = C.CDLL(p)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def synth() -> C.CDLL:
    global _synth
    if _synth is None:
        p = os.path.join(LIB_DIR, "libfa_synth.so")
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is missing: build it with `python -m ai_amd.build`")
        l = C.CDLL(p)
        for name, (res, args) in _SYNTH_SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _synth = l
    return _synth


def header_functions(path: str = HEADER) -> list[str]:
    """Names of the functions a header declares (for export checks)."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def check(ctx, rc: int) -> None:
    if rc != FA_OK:
        msg = lib().fa_last_error(ctx).decode()
        raise FaError(rc, msg)


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(vp)


# Objects that own library handles (contexts, models), closed in reverse
# creation order (models before the context they use) when the interpreter
# exits: the HIP runtime's own teardown runs after Python's, and streams,
# events or pinned buffers still live then (a program that never calls
# close()) made it abort.
_owners: list = []


def own(obj) -> None:
    """Registers obj (with a close() method) for closing at interpreter exit."""
    _owners[:] = [r for r in _owners if r() is not None]  # forget collected ones
    _owners.append(weakref.ref(obj))


@atexit.register
def _close_owners() -> None:
    for r in reversed(_owners):
        o = r()
        if o is not None:
            try:
                o.close()
            except Exception:
                pass
    _owners.clear()


class Context:
    """One GPU context (fa_ctx): a HIP stream plus scratch."""

    def __init__(self, device: int = 0):
        h = vp()
        rc = lib().fa_create(device, C.byref(h))
        if rc != FA_OK:
            raise FaError(rc, lib().fa_last_error(None).decode())
        self.h = h
        own(self)

    def close(self) -> None:
        if self.h:
            lib().fa_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return lib().fa_stream(self.h)

    def sync(self) -> None:
        check(self.h, lib().fa_sync(self.h))
