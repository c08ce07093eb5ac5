"""Seeded synthetic weights and inputs for the benchmark configurations.

The configurations (BASELINE.json "configs"): an EmbeddingGemma-300M-shaped
encoder with random-init weights (N(0, 0.02) rounded to bf16; norm weights
N(0, 0.1)) and token-id batches:

  C1  batch 1,   seq 128:  [BOS=2] + 127 uniform ids in [3, 262144)
  C2  batch 32,  seq 256:  lengths uniform in [64, 256], Zipf(1.1) ids, pad 0
  C3  batch 64,  seq 512:  all full length, uniform ids
  C4  batch 8,   seq 2048: lengths uniform in [1024, 2048], Zipf ids
  C5  batch 256, seq 128:  lengths uniform in [16, 128], Zipf ids; plus a
      corpus of 100 000 unit-norm float32 rows to score against

Every array comes from libfa_synth.so keyed by (seed, name), so the GPU path
and the CPU oracle see bit-identical inputs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _native as N

WEIGHT_SEED = 0xF1BE5EED
BOS, PAD = 2, 0


def normal_bf16(seed: int, name: str, std: float, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.uint16)
    N.synth().fa_synth_normal_bf16(seed, name.encode(), std, n, out.ctypes.data)
    return out.reshape(shape)


def normal_f32(seed: int, name: str, std: float, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    N.synth().fa_synth_normal_f32(seed, name.encode(), std, n, out.ctypes.data)
    return out.reshape(shape)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    N.synth().fa_bf16_to_f32(a.ctypes.data, a.size, out.ctypes.data)
    return out


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    N.synth().fa_f32_to_bf16(a.ctypes.data, a.size, out.ctypes.data)
    return out


def uniform_i32(seed: int, name: str, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    N.synth().fa_synth_uniform_i32(seed, name.encode(), lo, hi, n, out.ctypes.data)
    return out


def zipf_i32(seed: int, name: str, s: float, n_ranks: int, offset: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    rc = N.synth().fa_synth_zipf_i32(seed, name.encode(), s, n_ranks, offset, n, out.ctypes.data)
    if rc != 0:
        raise ValueError("zipf: n_ranks must be positive")
    return out


def unit_rows(seed: int, name: str, n: int, d: int) -> np.ndarray:
    out = np.empty((n, d), np.float32)
    N.synth().fa_synth_unit_rows(seed, name.encode(), n, d, out.ctypes.data)
    return out


# ---- model ----------------------------------------------------------------------

@dataclass
class ModelShape:
    """EmbeddingGemma-300M hyper-parameters (its config.json values, as models/gemma/config.go reads them)."""
    hidden_size: int = 768
    num_hidden_layers: int = 24
    num_attention_heads: int = 3
    num_key_value_heads: int = 1
    head_dim: int = 256
    intermediate_size: int = 1152
    vocab_size: int = 262144
    sliding_window: int = 512
    use_bidirectional: int = 1
    sliding_window_pattern: int = 6
    rope_local_base_freq: float = 1e4
    rope_theta: float = 1e6
    query_pre_attn_scalar: float = 256.0
    rms_norm_eps: float = 1e-6
    max_tokens: int = 2048
    dense_out: list = field(default_factory=lambda: [3072, 768])
    dense_act: list = field(default_factory=list)  # per Dense layer: 0 identity, 3 Tanh; empty: identity


def weight_specs(s: ModelShape):
    """(name, shape, kind) of every checkpoint tensor; kind 'm' = matrix
    N(0, 0.02) in bf16, 'n' = norm vector N(0, 0.1) in float32."""
    d, H, Hkv, D, F = s.hidden_size, s.num_attention_heads, s.num_key_value_heads, s.head_dim, s.intermediate_size
    specs = [("embed_tokens.weight", (s.vocab_size, d), "m")]
    for l in range(s.num_hidden_layers):
        p = f"layers.{l}."
        specs += [
            (p + "input_layernorm.weight", (d,), "n"),
            (p + "post_attention_layernorm.weight", (d,), "n"),
            (p + "pre_feedforward_layernorm.weight", (d,), "n"),
            (p + "post_feedforward_layernorm.weight", (d,), "n"),
            (p + "self_attn.q_norm.weight", (D,), "n"),
            (p + "self_attn.k_norm.weight", (D,), "n"),
            (p + "self_attn.q_proj.weight", (H * D, d), "m"),
            (p + "self_attn.k_proj.weight", (Hkv * D, d), "m"),
            (p + "self_attn.v_proj.weight", (Hkv * D, d), "m"),
            (p + "self_attn.o_proj.weight", (d, H * D), "m"),
            (p + "mlp.gate_proj.weight", (F, d), "m"),
            (p + "mlp.up_proj.weight", (F, d), "m"),
            (p + "mlp.down_proj.weight", (d, F), "m"),
        ]
    specs.append(("norm.weight", (d,), "n"))
    din = d
    for i, o in enumerate(s.dense_out):
        specs.append((f"dense.{i}.linear.weight", (o, din), "m"))
        din = o
    return specs


@dataclass
class ModelShape2:
    """EmbeddingGemma 2 text tower hyper-parameters (models/gemma/config.go:
    247-297; the values of the reference's TestConfig2, gemma2_test.go:44-95):
    layer l is full attention iff (l+1) % 6 == 0, with head_dim
    global_head_dim and global_kv_heads key/value heads; sliding layers use
    head_dim and num_key_value_heads and attend within an inclusive radius of
    sliding_window."""
    hidden_size: int = 512
    num_hidden_layers: int = 12
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 256
    global_head_dim: int = 512
    global_kv_heads: int = 1
    intermediate_size: int = 2048
    vocab_size: int = 262144
    sliding_window: int = 512
    hidden_size_per_layer_input: int = 512
    embedding_dim: int = 768
    rope_local_base_freq: float = 1e4
    rope_theta: float = 1e6
    rms_norm_eps: float = 1e-6
    max_tokens: int = 8192
    dense_out: list = field(default_factory=list)

    def sliding(self, l: int) -> bool:
        return (l + 1) % 6 != 0

    def layer_head_dim(self, l: int) -> int:
        return self.head_dim if self.sliding(l) else self.global_head_dim

    def layer_kv_heads(self, l: int) -> int:
        return self.num_key_value_heads if self.sliding(l) else self.global_kv_heads


def weight_specs2(s: ModelShape2):
    """(name, shape, kind) of every EmbeddingGemma 2 tensor (names without
    the checkpoint's "language_model." prefix, as models/gemma/model.go:
    142-205 reads them); kinds: 'm' matrix, 'g' RMSNorm gain (multiplies the
    normalised value directly), 's' the per-layer scalar."""
    d, H, F, P = s.hidden_size, s.num_attention_heads, s.intermediate_size, s.hidden_size_per_layer_input
    specs = [("embed_tokens.weight", (s.vocab_size, d), "m")]
    for l in range(s.num_hidden_layers):
        D, Hkv = s.layer_head_dim(l), s.layer_kv_heads(l)
        p = f"layers.{l}."
        specs += [
            (p + "input_layernorm.weight", (d,), "g"),
            (p + "post_attention_layernorm.weight", (d,), "g"),
            (p + "pre_feedforward_layernorm.weight", (d,), "g"),
            (p + "post_feedforward_layernorm.weight", (d,), "g"),
            (p + "self_attn.q_norm.weight", (D,), "g"),
            (p + "self_attn.k_norm.weight", (D,), "g"),
            (p + "self_attn.q_proj.weight", (H * D, d), "m"),
            (p + "self_attn.k_proj.weight", (Hkv * D, d), "m"),
            (p + "self_attn.v_proj.weight", (Hkv * D, d), "m"),
            (p + "self_attn.o_proj.weight", (d, H * D), "m"),
            (p + "mlp.gate_proj.weight", (F, d), "m"),
            (p + "mlp.up_proj.weight", (F, d), "m"),
            (p + "mlp.down_proj.weight", (d, F), "m"),
            (p + "ple_block.per_layer_input_gate.weight", (P, d), "m"),
            (p + "ple_block.per_layer_projection.weight", (d, P), "m"),
            (p + "ple_block.post_per_layer_input_norm.weight", (d,), "g"),
            (p + "layer_scalar", (1,), "s"),
        ]
    specs += [("norm.weight", (d,), "g"),
              ("ple.per_layer_model_projection.weight", (s.num_hidden_layers * P, d), "m"),
              ("ple.per_layer_projection_norm.weight", (P,), "g"),
              ("embedding_projection.weight", (s.embedding_dim, d), "m")]
    din = s.embedding_dim
    for i, o in enumerate(s.dense_out):
        specs.append((f"dense.{i}.linear.weight", (o, din), "m"))
        din = o
    return specs


def make_weight(name: str, shape, kind: str, seed: int = WEIGHT_SEED, mat_std: float = 0.02,
                norm_std: float = 0.1) -> np.ndarray:
    """bf16 bits (uint16) for matrices ('m', N(0, mat_std)); float32 for norm
    vectors ('n': N(0, norm_std), applied as 1+w), gains ('g': 1 + N(0,
    norm_std), applied as is) and layer scalars ('s': 1 + N(0, 0.1))."""
    if kind == "m":
        return normal_bf16(seed, name, mat_std, shape)
    if kind == "g":
        return (normal_f32(seed, name, norm_std, shape) + np.float32(1)).astype(np.float32)
    if kind == "s":
        return (normal_f32(seed, name, 0.1, shape) + np.float32(1)).astype(np.float32)
    return normal_f32(seed, name, norm_std, shape)


# ---- inputs ---------------------------------------------------------------------

@dataclass
class Batch:
    name: str
    ids: np.ndarray       # [B, T] int32, right-padded with PAD
    lengths: np.ndarray   # [B] int32
    corpus: np.ndarray | None = None  # C5 only: [100000, 768] float32

    @property
    def B(self) -> int:
        return self.ids.shape[0]

    @property
    def T(self) -> int:
        return self.ids.shape[1]

    @property
    def tokens(self) -> int:
        return int(self.lengths.sum())


CONFIGS = {
    "C1": dict(B=1, T=128, lengths=None, ids="uniform", seed=1),
    "C2": dict(B=32, T=256, lengths=(64, 256), ids="zipf", seed=2),
    "C3": dict(B=64, T=512, lengths=None, ids="uniform", seed=3),
    "C4": dict(B=8, T=2048, lengths=(1024, 2048), ids="zipf", seed=4),
    "C5": dict(B=256, T=128, lengths=(16, 128), ids="zipf", seed=5),
}


def make_batch(name: str, vocab: int = 262144, with_corpus: bool = True, n_docs: int = 100000,
               d: int = 768) -> Batch:
    c = CONFIGS[name]
    B, T, seed = c["B"], c["T"], c["seed"]
    if c["lengths"] is None:
        lengths = np.full(B, T, np.int32)
    else:
        lo, hi = c["lengths"]
        lengths = uniform_i32(seed, "lengths", lo, hi + 1, B)
    n = B * T
    if c["ids"] == "uniform":
        body = uniform_i32(seed, "ids", 3, vocab, n)
    else:
        body = zipf_i32(seed, "ids", 1.1, vocab - 3, 2, n)  # ranks 1..vocab-3 -> ids 3..vocab-1
    ids = body.reshape(B, T).copy()
    ids[:, 0] = BOS
    cols = np.arange(T)[None, :]
    ids[cols >= lengths[:, None]] = PAD
    corpus = None
    if name == "C5" and with_corpus:
        corpus = unit_rows(seed, "corpus", n_docs, d)
    return Batch(name, ids.astype(np.int32), lengths.astype(np.int32), corpus)
