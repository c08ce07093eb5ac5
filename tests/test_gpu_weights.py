"""Checkpoints the reference loads that are not bf16: float32 (and float16)
matrices whose values bf16 cannot hold, and Dense layers with a Tanh
activation; and the tensor.MatMulFused drop-in with float32 weights in the
reference's [k x n] layout.

gemma.Load converts F32, F16 and F64 tensors to float32
(safetensors/convert.go:23-55) and accepts a Dense layer whose activation is
torch.nn.modules.activation.Tanh (models/gemma/model.go:296-301). Such a
matrix is kept as three bf16 planes (hi + mid + lo = the float32 value) and
its products take six term products per operand pair; the oracle computes in
float32 from the same values. Bars as the encoder's: cosine >= 0.999999 and
max |delta| <= 1e-5 on the embeddings, products within 1e-4 (1 + |want|).
"""
import numpy as np
import pytest

import oracle_lib as O
from ai_amd import _native as N
from ai_amd import gemma as G
from ai_amd import synth as S
from ai_amd import tensor as T

pytestmark = pytest.mark.gpu


def small_shape(**kw):
    base = dict(num_hidden_layers=3, vocab_size=4096, sliding_window_pattern=3)
    base.update(kw)
    return S.ModelShape(**base)


def batch(shape, seed=3):
    r = np.random.default_rng(seed)
    lengths = np.array([300, 77, 1, 260, 140], np.int32)
    ids = np.zeros((len(lengths), 300), np.int32)
    for b, L in enumerate(lengths):
        ids[b, :L] = r.integers(3, shape.vocab_size, L)
        ids[b, 0] = 2
    return ids, lengths


def weights(shape, how):
    """name -> array: how(name, kind) picks, per matrix, 'bf16' (bits),
    'f32exact' (bf16 values as float32), 'f32' (N(0, 0.02) float32) or
    'f16' (float32 values that are float16 numbers)."""
    out = {}
    for name, shp, kind in S.weight_specs(shape):
        if kind != "m":
            out[name] = S.make_weight(name, shp, kind)
            continue
        h = how(name)
        if h == "bf16":
            out[name] = S.make_weight(name, shp, kind)
        elif h == "f32exact":
            out[name] = S.bf16_to_f32(S.make_weight(name, shp, kind))
        else:
            w = S.normal_f32(S.WEIGHT_SEED, name, 0.02, shp)
            out[name] = w.astype(np.float16).astype(np.float32) if h == "f16" else w
    return out


def run_pair(ctx, shape, ws):
    gm = G.Model(shape, ctx)
    om = O.OracleModel(shape)
    for name, w in ws.items():
        gm.set_weight(name, w)
        om.set(name, S.bf16_to_f32(w) if w.dtype == np.uint16 else w)
    gm.finalize()
    om.finalize()
    ids, lengths = batch(shape)
    got = gm.embed_ids(ids, lengths)
    want = om.embed(ids, lengths)
    states = []
    for n in (1, shape.num_hidden_layers):
        g = gm.encode_ids(ids, lengths, n_layers=n).astype(np.float64)
        w = om.encode(ids, lengths, layers=[n])[0].astype(np.float64)
        states.append((np.linalg.norm(g - w, axis=1) / np.linalg.norm(w, axis=1)).max())
    gm.close()
    om.close()
    return got, want, states


def check(got, want, states, what):
    c = (got.astype(np.float64) * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    d = np.abs(got.astype(np.float64) - want).max()
    print(f"{what}: cosine min={c.min():.9f} max|d|={d:.3g} hidden-state row rel err {max(states):.3g}", flush=True)
    assert c.min() >= 0.999999 and d <= 1e-5, what
    assert max(states) <= 1e-5, what


def test_float32_matrices_not_bf16_exact(ctx):
    """Every matrix, the embedding table included, in float32 with values
    bf16 cannot hold (gemma.Load accepts F32 checkpoints)."""
    shape = small_shape()
    got, want, st = run_pair(ctx, shape, weights(shape, lambda n: "f32"))
    check(got, want, st, "all float32")


def test_float16_valued_matrices(ctx):
    """Float16 checkpoints (convert.go's f16to32): 11-bit significands."""
    shape = small_shape()
    got, want, st = run_pair(ctx, shape, weights(shape, lambda n: "f16"))
    check(got, want, st, "float16 values")


def test_mixed_planes_in_stacked_matrices(ctx):
    """q bf16 then k float32 (q|k|v becomes three planes after q's rows are
    in), gate bf16-exact float32 and up float32 (interleaved gate|up), the
    down product and the head in bf16, the embedding float32."""
    shape = small_shape()

    def how(n):
        if "k_proj" in n or "up_proj" in n or n == "embed_tokens.weight":
            return "f32"
        if "gate_proj" in n:
            return "f32exact"
        return "bf16"
    got, want, st = run_pair(ctx, shape, weights(shape, how))
    check(got, want, st, "mixed planes")


def test_reupload_exact_rows_into_three_planes(ctx):
    """A matrix promoted to three planes and then set again from bf16 data:
    the mid and lo planes of those rows must be zeroed (no stale terms)."""
    shape = small_shape(num_hidden_layers=1, sliding_window_pattern=1)
    ws = weights(shape, lambda n: "bf16")
    gm = G.Model(shape, ctx)
    for name, w in ws.items():
        gm.set_weight(name, w)
    gm.set_weight("layers.0.self_attn.k_proj.weight", S.normal_f32(9, "noise", 0.02, (256, 768)))
    gm.set_weight("layers.0.self_attn.k_proj.weight", ws["layers.0.self_attn.k_proj.weight"])
    gm.finalize()
    om = O.OracleModel(shape)
    for name, w in ws.items():
        om.set(name, S.bf16_to_f32(w) if w.dtype == np.uint16 else w)
    om.finalize()
    ids, lengths = batch(shape)
    got, want = gm.embed_ids(ids, lengths), om.embed(ids, lengths)
    gm.close()
    om.close()
    check(got, want, [0.0], "re-set bf16 rows after float32")


@pytest.mark.parametrize("acts", [[3, 0], [0, 3], [3, 3]])
def test_tanh_dense_layers(ctx, acts):
    """Dense layers followed by Tanh (model.go:296-301, embed.go:415-418)."""
    shape = small_shape(dense_act=acts)
    got, want, st = run_pair(ctx, shape, weights(shape, lambda n: "bf16"))
    check(got, want, st, f"Tanh Dense {acts}")


@pytest.mark.parametrize("layout", [N.FA_B_KN, N.FA_B_NK])
@pytest.mark.parametrize("wdtype", ["f32", "bf16"])
def test_matmul_dropin_weights_at_the_gate_shape(ctx, layout, wdtype):
    """tensor.MatMulFused as the reference calls it for the GeGLU gate
    (embed.go:227): x [5517 x 768] . W [768 x 1152] with RowScale, GELU and
    Mul, W float32 (or bf16) in [k x n] (the Go weight layout) or [n x k]."""
    r = np.random.default_rng(5)
    m, k, n = 5517, 768, 1152
    a = r.standard_normal((m, k)).astype(np.float32)
    w = S.normal_f32(5, "gate_dropin", 0.02, (k, n))
    if wdtype == "bf16":
        wb = S.f32_to_bf16(w)
        w = S.bf16_to_f32(wb)
        wpass = wb if layout == N.FA_B_KN else np.ascontiguousarray(wb.T)
    else:
        wpass = w if layout == N.FA_B_KN else np.ascontiguousarray(w.T)
    rs = r.uniform(0.5, 1.5, m).astype(np.float32)
    mul = r.standard_normal((m, n)).astype(np.float32)
    got = T.MatMulFused(a, wpass, T.Fused(RowScale=rs, Act=T.GELUAct, Mul=mul), w_layout=layout, ctx=ctx)
    want = O.gemm(a, w, rowscale=rs, act=T.GELUAct, mul=mul)
    d = np.abs(got.astype(np.float64) - want)
    print(f"MatMulFused {wdtype} layout {layout}: max|d|={d.max():.3g}", flush=True)
    assert (d <= 1e-4 * (1 + np.abs(want))).all()


def test_matmul_tanh_activation(ctx):
    r = np.random.default_rng(6)
    a = r.standard_normal((64, 256)).astype(np.float32)
    w = (r.standard_normal((256, 96)) * 0.1).astype(np.float32)
    e = T.Fused(Act=N.FA_ACT_TANH)
    got = T.MatMulFused(a, w, e, ctx=ctx)
    want = O.tanh(O.gemm(a, w))
    assert np.abs(got - want).max() <= 1e-5


def test_three_plane_matrix_needs_whole_k_slabs(ctx):
    """A float32 matrix bfloat16 cannot hold runs on the six-term kernel,
    which takes 32-wide K slabs: an input width that is not a multiple of 32
    is refused when the weight is set (FA_ERR_UNSUPPORTED), not at the first
    embed; the same matrix with bf16-exact values is accepted (the fp32-MFMA
    kernel takes any width)."""
    shape = S.ModelShape(num_hidden_layers=1, vocab_size=256, dense_out=[100, 768])
    m = G.Model(shape, ctx)
    try:
        w = np.random.default_rng(5).standard_normal((768, 100)).astype(np.float32) * 0.02
        with pytest.raises(G.GemmaError, match=r"\[5\].*multiple of 32"):
            m.set_weight("dense.1.linear.weight", w)
        m.set_weight("dense.1.linear.weight", S.bf16_to_f32(S.f32_to_bf16(w)))
    finally:
        m.close()
