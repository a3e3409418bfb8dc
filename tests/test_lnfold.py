"""The LayerNorm fold on the host: the derived consts and the graph pass.

`fold_layernorm` rewrites LayerNorm -> linear as one `lnfold_matmul_epilogue`
op over the LayerNorm's input, with W' = fp16(ln_w * W) and bias2 = [c2 | c1]
derived from the feeds when the plan is staged. The GPU kernel's parity is in
tests/test_gpu_lnfold.py; here the algebra and the plan shape.
"""
from dataclasses import replace

import numpy as np
import pytest

from hexlib_amd import encoder as E
from hexlib_amd.exec import wholeplan as WP
from hexlib_amd.graph.fuse import fold_layernorm, fuse, fuse_residual, fuse_rope, lnfold_bias2, lnfold_weight


def _layernorm64(x, g, b, eps):
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


@pytest.mark.parametrize("seed", [0, 1])
def test_fold_identity_is_exact_when_the_scaled_weight_is(seed):
    """With LayerNorm gains that are powers of two, W' = fp16(g W) is exact, so
    rstd (x W' - mean c1) + c2 must equal LayerNorm(x) W + bias to float64
    rounding: a c2 without the ln_b W term, a c1 summed over W instead of W',
    or a sign slip each miss by orders of magnitude more."""
    r = np.random.default_rng(seed)
    M, Kd, N = 16, 256, 40
    x = r.standard_normal((M, Kd)) * 3.0 + 1.5
    g = 2.0 ** r.integers(0, 3, Kd)   # >= 1: g W stays an exact (normal) fp16
    b = r.standard_normal(Kd) * 0.3
    w = r.standard_normal((Kd, N)).astype(np.float16).astype(np.float64)
    bias = (r.standard_normal(N) * 0.1).astype(np.float32).astype(np.float64)
    wf = lnfold_weight(w, g).astype(np.float64)
    np.testing.assert_array_equal(wf, g[:, None] * w)
    b2 = lnfold_bias2(w, g, b, bias).astype(np.float64)
    c2, c1 = b2[:N], b2[N:]
    mean = x.mean(axis=1, keepdims=True)
    rstd = 1.0 / np.sqrt(x.var(axis=1, keepdims=True) + 1e-6)
    got = rstd * (x @ wf - mean * c1) + c2
    want = _layernorm64(x, g, b, 1e-6) @ w + bias
    # c1/c2 are stored as fp32: the only rounding left
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_bias2_layout():
    r = np.random.default_rng(3)
    w = r.standard_normal((64, 8)).astype(np.float16)
    g, b, bias = r.random(64) + 0.5, r.standard_normal(64), r.standard_normal(8)
    b2 = lnfold_bias2(w, g, b, bias)
    assert b2.dtype == np.float32 and b2.shape == (16,)
    np.testing.assert_allclose(b2[:8], bias + b @ w.astype(np.float64), rtol=1e-6)
    np.testing.assert_allclose(b2[8:], lnfold_weight(w, g).astype(np.float64).sum(axis=0), rtol=1e-6)


def _product_graph(cfg):
    g = E.build_vision_encoder(cfg)
    return fuse_residual(fuse_rope(fuse(g)))


def test_pass_folds_every_block_layernorm_of_the_batch1_plan():
    cfg = replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    g = _product_graph(cfg)
    n_ln = sum(op.kind == "layernorm" for op in g.ops)
    g2, derived = fold_layernorm(g, max_rows=256)
    assert not g2.problems()
    kinds = [op.kind for op in g2.ops]
    assert kinds.count("lnfold_matmul_epilogue") == 24
    assert kinds.count("layernorm") == n_ln - 24 == 1   # the merger's, read through a reshape
    assert len(derived) == 48
    for op in g2.ops:
        if op.kind != "lnfold_matmul_epilogue":
            continue
        x, wf, b2 = op.inputs[:3]
        assert g2.tensor(x).shape == (256, 768)
        assert g2.tensor(wf).const and g2.tensor(wf).dtype == "fp16"
        n = g2.tensor(wf).shape[1]
        assert g2.tensor(b2).shape == (2 * n,) and g2.tensor(b2).dtype == "fp32"
        assert op.attrs["eps"] == cfg.layernorm_eps
        assert len(op.inputs) == (5 if n == 2304 else 3)
    # above the row limit nothing changes
    g3, d3 = fold_layernorm(g, max_rows=255)
    assert g3 is g and d3 == {}


def test_plan_with_fold_stages_derived_consts():
    cfg_ref = replace(E.TINY_ENCODER, norm="layernorm", hidden_size=256, intermediate_size=512, num_heads=4)
    cfg = replace(cfg_ref, attention="fused_qkv_rope")
    g = E.build_vision_encoder(cfg)
    feeds = E.fuse_qkv_feeds(E.synthetic_feeds(E.build_vision_encoder(cfg_ref), cfg_ref, seed=1), cfg)
    plain = WP.build_whole_plan_batch(g, feeds, residual=True, rope=True)
    folded = WP.build_whole_plan_batch(g, feeds, residual=True, rope=True, fold_ln_rows=1 << 20)
    n_blocks = cfg.depth
    assert folded.n_ops == plain.n_ops - 2 * n_blocks
    specs = folded.op_specs
    assert specs.count("lnfold_matmul_epilogue_f16wt_rope") == n_blocks
    assert specs.count("lnfold_matmul_epilogue_f16wt") == n_blocks
    # the rope consumer's W' is staged pair-interleaved, the plain one transposed
    for op, spec in zip(folded.graph_ops, specs):
        if spec.startswith("lnfold"):
            lay = folded.placements[op.inputs[1]].layout
            assert lay == ("col_major_rope" if spec.endswith("rope") else "col_major")
            p = folded.placements[op.inputs[2]]
            assert p.dtype == "fp32" and p.nbytes == 4 * p.shape[0]
