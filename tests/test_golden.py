"""Golden vectors from an independent implementation (Hugging Face
transformers' Gemma3TextModel, tests/golden/make_gemma3_golden.py) pin the
whole encoder: the CPU oracle (CPU test) and the GPU path (gpu test) must
both reproduce them."""
import json
import os

import numpy as np
import pytest

import oracle_lib as O
from ai_amd import synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "gemma3_tiny.npz")


def load():
    z = np.load(GOLD, allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    shape = S.ModelShape(**meta["shape"])
    ws = {}
    for name, shp, kind in S.weight_specs(shape):
        if kind == "m":
            ws[name] = S.bf16_to_f32(S.normal_bf16(meta["seed"], name, meta["mat_std"], shp))
        else:
            ws[name] = S.normal_f32(meta["seed"], name, meta["norm_std"], shp)
    checksum = float(sum(np.float64(v).sum() for v in ws.values()))
    assert abs(checksum - meta["checksum"]) <= 1e-9 * max(1.0, abs(checksum)), "synthetic generator drifted"
    return shape, ws, z["ids"], z["lengths"], z["embeddings"], meta


def cos_rows(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


def test_oracle_matches_transformers_golden():
    shape, ws, ids, lengths, emb, meta = load()
    om = O.OracleModel(shape)
    for k, v in ws.items():
        om.set(k, v)
    om.finalize()
    got = om.embed(ids, lengths)
    c = cos_rows(got, emb)
    print(f"oracle vs {meta['source']}: cosine min {c.min():.8f}, max|d| {np.abs(got - emb).max():.3g}")
    assert c.min() >= 0.9999
    assert np.abs(got - emb).max() <= 1e-4


def test_float64_restatement_matches_transformers_golden():
    from test_oracle import f64_encoder
    shape, ws, ids, lengths, emb, _ = load()
    want = f64_encoder(shape, ws, ids, lengths)
    assert np.abs(want - emb).max() <= 1e-4


@pytest.mark.gpu
def test_gpu_matches_transformers_golden(ctx):
    from ai_amd import gemma as G
    shape, ws, ids, lengths, emb, meta = load()
    gm = G.Model(shape, ctx)
    for name, shp, kind in S.weight_specs(shape):
        gm.set_weight(name, S.f32_to_bf16(ws[name]) if kind == "m" else ws[name])
    gm.finalize()
    got = gm.embed_ids(ids, lengths)
    gm.close()
    c = cos_rows(got, emb)
    print(f"GPU vs {meta['source']}: cosine min {c.min():.8f}, max|d| {np.abs(got - emb).max():.3g}")
    assert c.min() >= 0.9999
    assert np.abs(got - emb).max() <= 1e-4
