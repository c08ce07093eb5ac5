"""Host-side mirror of fiber/ai's models/gemma API on the GPU encoder.

Model mirrors gemma.Model (models/gemma/model.go:40-71): it is created
empty, receives its checkpoint tensors by Hugging Face name (as gemma.Load
reads them from safetensors, model.go:142-191), and embeds token-id batches
(the ids-level core of (*Model).Embed, models/gemma/embed.go:15-157:
tokenisation is not on this path). Dim/Matryoshka truncation and errors
follow the reference (embed.go:24-30).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _native as N
from . import synth as S


class GemmaError(RuntimeError):
    """The error value gemma's functions return (the reference returns error)."""


def _config_struct(shape) -> N.GemmaConfig:
    if isinstance(shape, S.ModelShape2):
        return _config_struct2(shape)
    c = N.GemmaConfig()
    for f in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim",
              "intermediate_size", "vocab_size", "sliding_window", "use_bidirectional", "sliding_window_pattern",
              "max_tokens"):
        setattr(c, f, int(getattr(shape, f)))
    c.rope_local_base_freq = float(shape.rope_local_base_freq)
    c.rope_theta = float(shape.rope_theta)
    c.query_pre_attn_scalar = float(shape.query_pre_attn_scalar)
    c.rms_norm_eps = float(shape.rms_norm_eps)
    c.n_dense = len(shape.dense_out)
    for i, o in enumerate(shape.dense_out):
        c.dense_out[i] = int(o)
        c.dense_act[i] = int(shape.dense_act[i]) if i < len(shape.dense_act) else N.FA_ACT_NONE
    return c


def _config_struct2(s: S.ModelShape2) -> N.GemmaConfig:
    """EmbeddingGemma 2 (variant 2) geometry, per layer."""
    c = N.GemmaConfig()
    for f in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim",
              "intermediate_size", "vocab_size", "sliding_window", "max_tokens", "hidden_size_per_layer_input",
              "embedding_dim"):
        setattr(c, f, int(getattr(s, f)))
    c.variant = 2
    c.rope_local_base_freq = float(s.rope_local_base_freq)
    c.rope_theta = float(s.rope_theta)
    c.query_pre_attn_scalar = 1.0
    c.rms_norm_eps = float(s.rms_norm_eps)
    c.n_dense = len(s.dense_out)
    for i, o in enumerate(s.dense_out):
        c.dense_out[i] = int(o)
    for l in range(s.num_hidden_layers):
        c.layer_head_dim[l] = s.layer_head_dim(l)
        c.layer_kv_heads[l] = s.layer_kv_heads(l)
        c.layer_sliding[l] = 1 if s.sliding(l) else 0
    return c


class Model:
    def __init__(self, shape=None, ctx: N.Context | None = None):
        self.shape = shape or S.ModelShape()
        self.ctx = ctx or N.Context(0)
        self._cfg = _config_struct(self.shape)
        h = C.c_void_p()
        self._check(N.lib().fa_gemma_create(self.ctx.h, C.byref(self._cfg), C.byref(h)))
        self.h = h
        N.own(self)

    def _check(self, rc: int) -> None:
        if rc != N.FA_OK:
            raise GemmaError(f"[{rc}] {N.lib().fa_last_error(self.ctx.h).decode()}")

    def close(self) -> None:
        if getattr(self, "h", None):
            # a model outliving its context's close() cannot be destroyed
            # through it any more (the library's model keeps the context)
            if self.ctx.h:
                N.lib().fa_gemma_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def Dim(self) -> int:
        """Width of the embeddings (model.go:336-343)."""
        if self.shape.dense_out:
            return int(self.shape.dense_out[-1])
        if isinstance(self.shape, S.ModelShape2):
            return int(self.shape.embedding_dim)
        return int(self.shape.hidden_size)

    def set_weight(self, name: str, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data)
        if a.dtype == np.uint16:
            dt = N.FA_DT_BF16
        else:
            a = np.ascontiguousarray(a, dtype=np.float32)
            dt = N.FA_DT_F32
        shape = (C.c_int64 * a.ndim)(*a.shape)
        self._check(N.lib().fa_gemma_set_weight(self.h, name.encode(), dt, shape, a.ndim, a.ctypes.data))

    def finalize(self) -> None:
        self._check(N.lib().fa_gemma_finalize(self.h))

    def load_synthetic(self, seed: int = S.WEIGHT_SEED) -> None:
        """Random-init weights of the benchmark configuration, tensor by tensor."""
        specs = S.weight_specs2(self.shape) if isinstance(self.shape, S.ModelShape2) else S.weight_specs(self.shape)
        for name, shp, kind in specs:
            self.set_weight(name, S.make_weight(name, shp, kind, seed))
        self.finalize()

    def embed_ids(self, ids: np.ndarray, lengths: np.ndarray, dim: int = 0) -> np.ndarray:
        """[B, dim] L2-normalised embeddings of right-padded ids [B, T]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        lengths = np.ascontiguousarray(lengths, dtype=np.int32)
        if ids.ndim != 2 or lengths.shape != (ids.shape[0],):
            raise GemmaError(f"gemma: ids {list(ids.shape)} and lengths {list(lengths.shape)} do not match")
        B, T = ids.shape
        full = self.Dim()
        d = full if dim == 0 else dim
        if d < 1 or d > full:
            raise GemmaError(f"gemma: Dim({dim}) outside 1..{full}")
        out = np.empty((B, d), np.float32)
        self._check(N.lib().fa_gemma_embed_ids(self.h, ids.ctypes.data, lengths.ctypes.data, B, T, d,
                                               out.ctypes.data))
        return out

    def encode_ids(self, ids: np.ndarray, lengths: np.ndarray, n_layers: int = -1) -> np.ndarray:
        """Hidden states [sum(lengths), hidden] of the valid tokens, packed in
        batch order: the final ones (n_layers < 0, as (*Model).encode returns
        them, embed.go:160-240) or the residual stream after n_layers layers."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        lengths = np.ascontiguousarray(lengths, dtype=np.int32)
        if ids.ndim != 2 or lengths.shape != (ids.shape[0],):
            raise GemmaError(f"gemma: ids {list(ids.shape)} and lengths {list(lengths.shape)} do not match")
        B, T = ids.shape
        out = np.empty((int(lengths.astype(np.int64).sum()), int(self.shape.hidden_size)), np.float32)
        self._check(N.lib().fa_gemma_encode_ids(self.h, ids.ctypes.data, lengths.ctypes.data, B, T, n_layers,
                                                out.ctypes.data))
        return out

    def embed_ids_dev(self, d_ids: int, lengths: np.ndarray, B: int, T: int, d_out: int, dim: int = 0) -> None:
        """Enqueue the forward pass on device-resident ids/outputs (no sync)."""
        lengths = np.ascontiguousarray(lengths, dtype=np.int32)
        self._check(N.lib().fa_gemma_embed_ids_dev(self.h, d_ids, lengths.ctypes.data, B, T, dim, d_out))

    # profiling
    def set_profiling(self, on: bool) -> None:
        self._check(N.lib().fa_gemma_set_profiling(self.h, 1 if on else 0))

    def reset_stats(self) -> None:
        self._check(N.lib().fa_gemma_reset_stats(self.h))

    def kernel_stats(self) -> dict:
        out = {}
        for kind, name in enumerate(N.KERNEL_KINDS):
            n = C.c_int64()
            ms, fl, by = C.c_double(), C.c_double(), C.c_double()
            self._check(N.lib().fa_gemma_kernel_stats(self.h, kind, C.byref(n), C.byref(ms), C.byref(fl),
                                                      C.byref(by)))
            out[name] = dict(launches=n.value, ms=ms.value, flops=fl.value, bytes=by.value)
        return out
