"""Pins the CPU oracle (oracle/fa_oracle.cpp) before it is trusted as the
parity checker. CPU only.

Each oracle function is checked against what the reference's own tests
assert and against what the mathematics fixes, with inputs chosen so that a
plausible slip (a dropped term, a wrong sign or index, a swapped operand, a
reordered epilogue) fails:

  orc_exp              TestExpAccuracy, TestExpFlushesBelowClamp
                       (internal/kernel/kernel_test.go:311-352, exp_flush_test.go:11-45)
  orc_tanh             TestTanhAccuracy (kernel_test.go:378-408)
  orc_gelu             TestGELUAgainstFloat64 (kernel_test.go:441-463)
  orc_row_sum_squares  TestRowSumSquares KAT (tensor/matmul_fused_test.go:62-71)
  orc_rms_scale        closed form in float64
  orc_rmsnorm          TestRMSNormAndGradient / TestRMSNormFusedMatchesComposed
                       (tensor/attention_test.go:120-137, rope_test.go:83-102)
  orc_rope             TestRoPEKnown, TestRoPEPreservesNorm (rope_test.go:9-38),
                       plus the complex-rotation closed form
  orc_*_mask           TestWindowMask (rope_test.go:66-81), closed forms
  orc_gemm             refGemm float64 on the reference's shape list
                       (internal/blas/gemm_test.go:22-79) and the epilogue cases
                       (internal/blas/epilogue_test.go:12-110)
  orc_attention        naiveAttention float64 (tensor/attention_test.go:12-92),
                       exact zeros (attention_test.go:266-285), GQA, window
  orc_similarities_topk  brute-force sort, ties -> lower index (tensor/reduce.go:286-289)
  orc_model_embed      an independent float64 numpy restatement of the encoder
                       (tiny config), padding/batch invariance
                       (models/gemma/gemma_test.go:117-135), and golden vectors
                       from Hugging Face transformers' Gemma3 encoder
                       (tests/test_golden.py)
"""
import math

import numpy as np
import pytest

import oracle_lib as O

MASK_NEG = -1e9


def close_enough(got, want, tol):
    """internal/kernel/kernel_test.go:37-39."""
    return np.abs(np.asarray(got, np.float64) - want) <= tol * (1 + np.abs(want))


# ---- element-wise math -----------------------------------------------------------

@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 15, 16, 17, 1000, 4097])
def test_exp_accuracy(n):
    x = (-90 + 180 * np.arange(n, dtype=np.float32) / np.float32(max(1, n - 1))).astype(np.float32)
    z = O.exp(x)
    below = x < -87.0
    assert np.all(z[below] == 0)
    xc = np.minimum(x[~below], np.float32(88.3762626647949)).astype(np.float64)
    want = np.exp(xc)
    rel = np.abs(z[~below].astype(np.float64) - want) / want
    assert rel.size == 0 or rel.max() <= 3e-7
    assert np.all(np.isfinite(z))


def test_exp_special_and_flush():
    z = O.exp(np.array([0, np.inf, -np.inf], np.float32))
    assert z[0] == 1 and z[1] >= 1e38 and z[2] <= 1e-37
    x = np.array([-1e9, -87.0001, -86.9] + [i * 0.25 for i in range(3, 20)], np.float32)
    z = O.exp(x)
    bits = z.view(np.uint32)
    assert bits[0] == 0 and bits[1] == 0
    assert (bits[2] & 0x7F800000) != 0  # a normal, not a denormal
    assert abs(z[2] - np.float32(math.exp(-86.9))) <= 2e-6 * z[2]


@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 15, 16, 17, 1000, 4097])
def test_tanh_accuracy(n):
    x = (-12 + 24 * np.arange(n, dtype=np.float32) / np.float32(max(1, n - 1))).astype(np.float32)
    if n == 4097:
        x[:1024] = (-1e-3 + 2e-3 * np.arange(1024, dtype=np.float32) / np.float32(1023)).astype(np.float32)
    z = O.tanh(x).astype(np.float64)
    want = np.tanh(x.astype(np.float64))
    assert np.all(np.abs(z - want) <= 2e-6 * np.abs(want) + 1e-7)
    s = O.tanh(np.array([0, np.inf, -np.inf], np.float32))
    assert s.tolist() == [0, 1, -1]


def test_gelu_against_float64():
    x = (-8 + 16 * np.arange(5000, dtype=np.float32) / np.float32(4999)).astype(np.float32)
    z = O.gelu(x)
    fv = x.astype(np.float64)
    u = 0.7978845608028654 * (fv + 0.044715 * fv ** 3)
    want = 0.5 * fv * (1 + np.tanh(u))
    assert np.all(close_enough(z, want, 1e-5))
    # the erf GELU differs by up to ~1e-3: the tanh form is pinned, not just "a GELU"
    from scipy.special import erf
    werf = 0.5 * fv * (1 + erf(fv / math.sqrt(2)))
    assert np.abs(z - werf).max() > 1e-4


# ---- row statistics ------------------------------------------------------------------

def test_row_sum_squares_kat():
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    assert O.row_sum_squares(x).tolist() == [14, 77]
    assert O.row_sum_squares(np.ascontiguousarray(x.T)).tolist() == [17, 29, 45]


def test_rms_scale_closed_form():
    ss = np.array([0, 1, 14, 77, 1e-3, 5e4], np.float32)
    got = O.rms_scale(ss, 768, 1e-6)
    want = 1 / np.sqrt(ss.astype(np.float64) / 768 + 1e-6)
    assert np.all(np.abs(got - want) <= 1e-7 * want)


def test_rmsnorm_closed_form_and_composed():
    r = np.random.default_rng(3)
    x = (r.standard_normal((4, 6)) * 2).astype(np.float32)
    g = (r.random(6) + 0.5).astype(np.float32)
    y = O.rmsnorm(x, g, 1e-6)
    rms = np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    want = x / rms * g
    assert np.abs(y - want).max() <= 1e-5
    for shp in [(4, 5, 64), (2, 3, 8, 16)]:
        x = r.standard_normal(shp).astype(np.float32)
        g = r.standard_normal(shp[-1]).astype(np.float32)
        y = O.rmsnorm(x, g, 1e-6)
        comp = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * g
        assert np.all(np.abs(y - comp) <= 1e-6 + 1e-5 * np.abs(comp))


# ---- RoPE ---------------------------------------------------------------------------------

def test_rope_known():
    got = O.rope(np.array([[1, 0]], np.float32), 10000, [1])
    assert abs(got[0, 0] - math.cos(1)) <= 1e-6 and abs(got[0, 1] - math.sin(1)) <= 1e-6
    ident = O.rope(np.array([[3, -4, 5, 6]], np.float32), 10000, [0])
    assert np.abs(ident - [[3, -4, 5, 6]]).max() <= 1e-6


def test_rope_norm_and_complex_closed_form():
    r = np.random.default_rng(1)
    x = r.standard_normal((2, 3, 8, 16)).astype(np.float32)
    pos = [0, 5, 9, 100, 500, 1000, 3, 7]
    y = O.rope(x, 1e6, pos)
    xn, yn = (x.astype(np.float64) ** 2).sum(-1), (y.astype(np.float64) ** 2).sum(-1)
    assert np.all(np.abs(xn - yn) <= 1e-3 * (xn + 1))
    # rotate-half as a complex rotation of (x_i + i x_{i+D/2}) by t * base^(-2i/D)
    D = 16
    z = x[..., :D // 2].astype(np.float64) + 1j * x[..., D // 2:].astype(np.float64)
    ang = np.array(pos, np.float64)[:, None] * 1e6 ** (-np.arange(0, D, 2) / D)[None, :]
    w = z * np.exp(1j * ang)
    want = np.concatenate([w.real, w.imag], -1)
    assert np.abs(y - want).max() <= 1e-5


# ---- masks ------------------------------------------------------------------------------

def test_masks():
    m = O.window_mask(5, 2)
    for i in range(5):
        for j in range(5):
            assert m[i, j] == (MASK_NEG if abs(i - j) >= 2 else 0)
    p = O.padding_mask([3, 0, 5], 5)
    assert p.shape == (3, 1, 1, 5)
    assert p[0, 0, 0].tolist() == [0, 0, 0, MASK_NEG, MASK_NEG]
    assert np.all(p[1] == MASK_NEG) and np.all(p[2] == 0)
    c = O.causal_mask(4)
    assert np.array_equal(c != 0, np.triu(np.ones((4, 4), bool), 1))


# ---- GEMM + epilogue ----------------------------------------------------------------------

REF_SHAPES = [(1, 1, 1), (1, 1, 100), (1, 17, 5), (1, 100, 300), (5, 1, 7), (300, 1, 100), (3, 3, 3), (4, 16, 1),
              (6, 16, 7), (8, 12, 3), (12, 32, 9), (13, 33, 9), (5, 17, 9), (7, 37, 19), (64, 64, 64),
              (129, 65, 33), (133, 257, 300), (100, 20, 513), (257, 33, 1), (31, 4097, 7), (300, 300, 300)]


@pytest.mark.parametrize("m,n,k", REF_SHAPES)
def test_gemm_vs_float64(m, n, k):
    r = np.random.default_rng(m * 7 + n * 3 + k)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(close_enough(O.gemm(a, b), want, 1e-4))


def _epi_ref(a, b, bias=None, rs=None, act=0, mul=None, res=None):
    y = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32).astype(np.float64)
    if bias is not None:
        y = y + bias
    if rs is not None:
        y = y * rs[:, None]
    if act == 1:
        y = np.maximum(y, 0)
    elif act == 2:
        y = 0.5 * y * (1 + np.tanh(0.7978845608028654 * (y + 0.044715 * y ** 3)))
    if mul is not None:
        y = y * mul
    if res is not None:
        y = y + res
    return y


@pytest.mark.parametrize("m,k,n", [(1, 64, 300), (5, 700, 3), (33, 130, 77), (64, 1100, 96), (200, 64, 1), (7, 5, 9)])
def test_gemm_epilogue_cases(m, k, n):
    """internal/blas/epilogue_test.go:61-96 case list."""
    r = np.random.default_rng(m + k + n)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = r.random(n).astype(np.float32)
    rs = (0.5 + r.random(m)).astype(np.float32)
    mul = r.uniform(-1, 1, (m, n)).astype(np.float32)
    res = r.uniform(-1, 1, (m, n)).astype(np.float32)
    cases = [dict(bias=bias), dict(act=1), dict(act=2), dict(bias=bias, act=1), dict(rs=rs, act=2, mul=mul),
             dict(bias=bias, rs=rs, act=2, mul=mul, res=res), dict(res=res)]
    for c in cases:
        got = O.gemm(a, b, bias=c.get("bias"), rowscale=c.get("rs"), act=c.get("act", 0), mul=c.get("mul"),
                     residual=c.get("res"))
        want = _epi_ref(a, b, **c)
        assert np.all(close_enough(got, want, 1e-4)), c
    # order matters: RowScale after Bias (scale*(y+b), not scale*y+b)
    got = O.gemm(a, b, bias=bias, rowscale=rs)
    wrong = (a.astype(np.float64) @ b) * rs[:, None] + bias
    if m > 1 and n > 1:
        assert not np.all(close_enough(got, wrong, 1e-4))


# ---- attention -----------------------------------------------------------------------------

def naive_attention(q, k, v, mask, scale):
    """tensor/attention_test.go:12-43 in float64 over [B,H,T,D]."""
    s = np.einsum("bhtd,bhsd->bhts", q.astype(np.float64), k.astype(np.float64)) * scale
    if mask is not None:
        s = s + np.asarray(mask, np.float64)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhts,bhsd->bhtd", p, v.astype(np.float64))


def test_attention_matches_naive():
    r = np.random.default_rng(41)
    B, H, T, S, D = 2, 3, 5, 7, 4
    q, k, v = (r.standard_normal((B, H, n, D)).astype(np.float32) for n in (T, S, S))
    for mask in (None, O.padding_mask([S, 3], S)):
        got = O.attention(q, k, v, mask, 1 / math.sqrt(D))
        assert np.abs(got - naive_attention(q, k, v, mask, 1 / math.sqrt(D))).max() <= 1e-4


def test_attention_gqa_window_d256():
    r = np.random.default_rng(2)
    B, H, T, D = 2, 3, 40, 256
    q = r.standard_normal((B, H, T, D)).astype(np.float32)
    k1 = r.standard_normal((B, 1, T, D)).astype(np.float32)
    v1 = r.standard_normal((B, 1, T, D)).astype(np.float32)
    k, v = np.broadcast_to(k1, (B, H, T, D)), np.broadcast_to(v1, (B, H, T, D))
    lengths = [40, 23]
    mask = O.padding_mask(lengths, T) + O.window_mask(T, 9).reshape(1, 1, T, T)
    got = O.attention(q, k, v, mask, 0.0625)
    want = naive_attention(q, k, v, mask, 0.0625)
    # rows whose keys are all masked (padding queries far from any valid
    # key) are discarded by the model; float32 and float64 legitimately
    # disagree there (the -1.6e10 offset absorbs the scores in float32)
    for b, L in enumerate(lengths):
        assert np.abs(got[b, :, :L] - want[b, :, :L]).max() <= 1e-4
    # a swapped GQA mapping (each head its own keys) must not pass
    k2 = r.standard_normal((B, H, T, D)).astype(np.float32)
    assert np.abs(got[0] - naive_attention(q, k2, v, mask, 0.0625)[0]).max() > 1e-2


def test_masked_weights_exact_zero():
    r = np.random.default_rng(11)
    n, d = 64, 16
    q, k, v = (r.standard_normal((1, 1, n, d)).astype(np.float32) for _ in range(3))
    out = O.attention(q, k, v, O.causal_mask(n), 0.25)
    assert np.abs(out[0, 0, 0] - v[0, 0, 0]).max() <= 1e-6


# ---- similarities + top-k --------------------------------------------------------------------

def test_similarities_topk_bruteforce():
    r = np.random.default_rng(5)
    q = r.standard_normal((7, 32)).astype(np.float32)
    docs = r.standard_normal((500, 32)).astype(np.float32)
    docs[[10, 20, 30]] = docs[5]  # exact ties
    q[0] = docs[5]
    idx, val = O.similarities_topk(q, docs, 10)
    s = np.einsum("qd,nd->qn", q, docs)  # float32 like the oracle's dot
    for i in range(7):
        order = np.lexsort((np.arange(500), -s[i]))[:10]
        assert idx[i].tolist() == order.tolist()
    assert idx[0, :4].tolist() == [5, 10, 20, 30]


def test_similarities_topk_nan_rule():
    """NaN scores rank below every number (never selected while a number
    remains), whatever their position, the first included; slots past a
    row's non-NaN scores hold index -1. A mistake such as NaN-first order or
    the reference Argmax's "first element wins when it is NaN" fails here."""
    r = np.random.default_rng(6)
    q = r.standard_normal((2, 8)).astype(np.float32)
    docs = r.standard_normal((12, 8)).astype(np.float32)
    docs[[0, 4, 9]] = np.nan
    idx, val = O.similarities_topk(q, docs, 12)
    s = q.astype(np.float64) @ docs.T.astype(np.float64)
    for i in range(2):
        ok = [j for j in np.lexsort((np.arange(12), -np.nan_to_num(s[i], nan=-np.inf))) if not np.isnan(s[i, j])]
        assert idx[i, :9].tolist() == ok
        assert idx[i, 9:].tolist() == [-1, -1, -1]
        assert np.isnan(val[i, 9:]).all()
    idx1, _ = O.similarities_topk(q, docs, 1)
    assert idx1[:, 0].tolist() == [int(np.nanargmax(s[i])) for i in range(2)]


# ---- the encoder -----------------------------------------------------------------------------

def f64_encoder(shape, weights, ids, lengths, dim=0, states=None):
    """Independent float64 restatement of models/gemma/embed.go:160-240,381-475
    over unpadded sequences (one at a time), with unfolded weights. With a
    list `states`, appends per sequence the residual stream after 0, 1, ...
    layers followed by the final normed hidden states."""
    d, H, Hkv, D = shape.hidden_size, shape.num_attention_heads, shape.num_key_value_heads, shape.head_dim
    w = {k: v.astype(np.float64) for k, v in weights.items()}
    wb = shape.sliding_window // 2 + 1 if shape.use_bidirectional else shape.sliding_window
    outs = []
    for b in range(ids.shape[0]):
        L = int(lengths[b])
        x = w["embed_tokens.weight"][ids[b, :L]] * np.float64(np.float32(math.sqrt(d)))

        def rms(v, g):
            return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + shape.rms_norm_eps) * (1 + g)

        pos = np.arange(L)
        seq_states = [x.copy()]
        for l in range(shape.num_hidden_layers):
            p = f"layers.{l}."
            sliding = (l + 1) % shape.sliding_window_pattern != 0
            base = shape.rope_local_base_freq if sliding else shape.rope_theta
            h = rms(x, w[p + "input_layernorm.weight"])
            q = (h @ w[p + "self_attn.q_proj.weight"].T).reshape(L, H, D)
            k = (h @ w[p + "self_attn.k_proj.weight"].T).reshape(L, Hkv, D)
            v = (h @ w[p + "self_attn.v_proj.weight"].T).reshape(L, Hkv, D)
            q = rms(q, w[p + "self_attn.q_norm.weight"])
            k = rms(k, w[p + "self_attn.k_norm.weight"])
            inv = base ** (-np.arange(0, D, 2) / D)
            ang = pos[:, None] * inv[None, :]
            c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

            def rot(t):
                t1, t2 = t[..., :D // 2], t[..., D // 2:]
                return np.concatenate([t1 * c - t2 * s, t1 * s + t2 * c], -1)

            q, k = rot(q), rot(k)
            att = np.zeros((L, H, D))
            allowed = np.ones((L, L), bool)
            if sliding and shape.sliding_window > 0:
                allowed = np.abs(pos[:, None] - pos[None, :]) < wb
            for hh in range(H):
                kv = hh // (H // Hkv)
                sc = q[:, hh] @ k[:, kv].T / math.sqrt(shape.query_pre_attn_scalar)
                sc = np.where(allowed, sc, -np.inf)
                sc -= sc.max(1, keepdims=True)
                pr = np.exp(sc)
                pr /= pr.sum(1, keepdims=True)
                att[:, hh] = pr @ v[:, kv]
            o = att.reshape(L, H * D) @ w[p + "self_attn.o_proj.weight"].T
            x = x + rms(o, w[p + "post_attention_layernorm.weight"])
            h = rms(x, w[p + "pre_feedforward_layernorm.weight"])
            gt = h @ w[p + "mlp.gate_proj.weight"].T
            up = h @ w[p + "mlp.up_proj.weight"].T
            gu = 0.5 * gt * (1 + np.tanh(0.7978845608028654 * (gt + 0.044715 * gt ** 3))) * up
            x = x + rms(gu @ w[p + "mlp.down_proj.weight"].T, w[p + "post_feedforward_layernorm.weight"])
            seq_states.append(x.copy())
        hfin = rms(x, w["norm.weight"])
        if states is not None:
            states.append(seq_states + [hfin])
        y = hfin.mean(0)
        for i in range(len(shape.dense_out)):
            y = w[f"dense.{i}.linear.weight"] @ y
            if i < len(shape.dense_act) and shape.dense_act[i] == 3:  # Tanh Dense (model.go:296-301)
                y = np.tanh(y)
        if dim:
            y = y[:dim]
        outs.append(y / math.sqrt((y ** 2).sum() + 1e-12))
    return np.array(outs)


def tiny_shape(**kw):
    from ai_amd import synth as S
    base = dict(hidden_size=64, num_hidden_layers=3, num_attention_heads=3, num_key_value_heads=1, head_dim=32,
                intermediate_size=96, vocab_size=300, sliding_window=12, sliding_window_pattern=3,
                max_tokens=64, dense_out=[128, 64])
    base.update(kw)
    return S.ModelShape(**base)


def tiny_weights(shape, seed=7):
    from ai_amd import synth as S
    ws = {}
    for name, shp, kind in S.weight_specs(shape):
        # larger matrix scale than the real init, so every block moves the result
        w = S.normal_bf16(seed, name, 0.15, shp) if kind == "m" else S.normal_f32(seed, name, 0.3, shp)
        ws[name] = S.bf16_to_f32(w) if kind == "m" else w
    return ws


def oracle_model(shape, ws):
    om = O.OracleModel(shape)
    for k, v in ws.items():
        om.set(k, v)
    om.finalize()
    return om


@pytest.fixture(scope="module")
def tiny():
    shape = tiny_shape()
    ws = tiny_weights(shape)
    r = np.random.default_rng(0)
    lengths = np.array([20, 9, 1, 14], np.int32)
    ids = np.zeros((4, 20), np.int32)
    for b, L in enumerate(lengths):
        ids[b, :L] = r.integers(3, shape.vocab_size, L)
        ids[b, 0] = 2
    return shape, ws, ids, lengths


def cos_rows(a, b):
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


def test_oracle_encoder_vs_float64(tiny):
    shape, ws, ids, lengths = tiny
    om = oracle_model(shape, ws)
    got = om.embed(ids, lengths)
    want = f64_encoder(shape, ws, ids, lengths)
    assert np.abs(got - want).max() <= 1e-4
    assert cos_rows(got.astype(np.float64), want).min() >= 0.99999
    # Matryoshka: truncation before L2
    got = om.embed(ids, lengths, dim=40)
    want = f64_encoder(shape, ws, ids, lengths, dim=40)
    assert np.abs(got - want).max() <= 1e-4


def test_oracle_encoder_detects_window_and_base(tiny):
    """A wrong window bound or RoPE base must move the result: the pins above
    are sensitive to them."""
    shape, ws, ids, lengths = tiny
    want = f64_encoder(shape, ws, ids, lengths)
    for bad in (tiny_shape(use_bidirectional=0), tiny_shape(rope_theta=1e4), tiny_shape(sliding_window_pattern=2)):
        alt = f64_encoder(bad, ws, ids, lengths)
        assert np.abs(alt - want).max() > 1e-3


def test_oracle_padding_and_batch_invariance(tiny):
    """models/gemma/gemma_test.go:117-135: a sentence alone or padded in a batch."""
    shape, ws, ids, lengths = tiny
    om = oracle_model(shape, ws)
    full = om.embed(ids, lengths)
    for i in range(ids.shape[0]):
        L = int(lengths[i])
        alone = om.embed(ids[i:i + 1, :L], lengths[i:i + 1])
        assert cos_rows(alone.astype(np.float64), full[i:i + 1].astype(np.float64)).min() >= 0.9999
    # more padding columns than any sequence needs
    wide = np.zeros((ids.shape[0], 37), np.int32)
    wide[:, :20] = ids
    assert cos_rows(om.embed(wide, lengths).astype(np.float64), full.astype(np.float64)).min() >= 0.9999


def test_oracle_encode_states_vs_float64(tiny):
    """orc_model_encode's snapshots (the residual stream after each layer and
    the final hidden states) against the float64 restatement's, layer by
    layer; snapshot 0 is the gather times float32(sqrt(d)) exactly, and pooling
    the final states reproduces orc_model_embed."""
    shape, ws, ids, lengths = tiny
    om = oracle_model(shape, ws)
    nl = shape.num_hidden_layers
    st = []
    f64_encoder(shape, ws, ids, lengths, states=st)
    snaps = om.encode(ids, lengths, layers=list(range(nl + 1)) + [-1])
    rows = np.concatenate([np.arange(int(L)) + b * ids.shape[1] for b, L in enumerate(lengths)])
    want0 = ws["embed_tokens.weight"][ids.reshape(-1)[rows]] * np.float32(math.sqrt(shape.hidden_size))
    assert np.array_equal(snaps[0], want0.astype(np.float32))
    for i in range(nl + 2):
        ref = np.concatenate([s[i] for s in st])
        err = np.abs(snaps[i] - ref).max() / np.abs(ref).max()
        assert err < 2e-5, (i, err)
    # pool + head + L2 of the final states in float64 against orc_model_embed
    h = snaps[-1].astype(np.float64)
    off = np.concatenate([[0], np.cumsum(lengths)])
    y = np.stack([h[off[b]:off[b + 1]].mean(0) for b in range(len(lengths))])
    for i in range(len(shape.dense_out)):
        y = y @ ws[f"dense.{i}.linear.weight"].astype(np.float64).T
    y /= np.linalg.norm(y, axis=1, keepdims=True)
    assert np.abs(om.embed(ids, lengths) - y).max() < 1e-6
    with pytest.raises(ValueError):
        om.encode(ids, lengths, layers=[nl + 1])


def test_oracle_tanh_dense_head(tiny):
    """A Dense layer with a Tanh activation (model.go:296-301, applied after
    the product, embed.go:415-418) against the float64 restatement; dropping
    the Tanh must move the result."""
    shape, ws, ids, lengths = tiny
    sh = tiny_shape(dense_act=[3, 0])
    om = oracle_model(sh, ws)
    got = om.embed(ids, lengths)
    want = f64_encoder(sh, ws, ids, lengths)
    assert np.abs(got - want).max() <= 1e-4
    plain = f64_encoder(shape, ws, ids, lengths)
    assert np.abs(plain - want).max() > 1e-3
