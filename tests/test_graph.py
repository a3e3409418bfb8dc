"""Graph, fusion, dispatch-table and whole-plan invariants (CPU).

Restates the reference's coverage tests (`hexlib/tests/test_encoder_dispatch_coverage.py`,
`test_runtime_genentry.py`, `test_pass_fuse.py`, `test_wholeplan.py:44-160`).
"""
import collections

import numpy as np
import pytest

from hexlib_amd import encoder as E
from hexlib_amd.exec import wholeplan as WP
from hexlib_amd.exec.runner import KIND_ID, SPECS, SelectError, select
from hexlib_amd.graph.fuse import fuse
from hexlib_amd.graph.ir import Graph, Op, Tensor


@pytest.fixture(scope="module")
def qwen_fused():
    return fuse(E.build_vision_encoder(E.QWEN35_VISION_Q4))


def test_plan_is_the_reference_size(qwen_fused):
    kinds = collections.Counter(op.kind for op in qwen_fused.ops)
    assert len(qwen_fused.ops) == 308
    assert kinds["reshape"] == 49
    assert kinds["matmul"] == 24
    assert kinds["matmul_epilogue"] == 75


def test_every_non_reshape_op_selects_a_kernel(qwen_fused):
    for op in qwen_fused.ops:
        if op.kind == "reshape":
            continue
        dtypes = [qwen_fused.tensor(n).dtype for n in op.inputs]
        select(op.kind, dict(op.attrs), dtypes)


def test_shipped_kind_ids_never_move():
    assert {k: KIND_ID[k] for k in list(KIND_ID)[:12]} == {
        "add": 1, "cast": 2, "layernorm": 3, "matmul": 4, "matmul_epilogue": 5,
        "patchify": 6, "reshape": 7, "rope_2d": 8, "scale": 9, "softmax": 10,
        "transpose": 11, "transpose_hd": 12}
    assert len(set(KIND_ID.values())) == len(KIND_ID)


def test_every_spec_has_a_kind_id():
    assert set(SPECS) <= set(KIND_ID)


def test_variant_selection():
    assert select("transpose", {"perm": (1, 0, 2)})[0] == "transpose"
    assert select("transpose", {"perm": (0, 2, 1)})[0] == "transpose_hd"
    assert select("transpose", {"perm": (0, 2, 1, 3)})[0] == "transpose_bth"
    with pytest.raises(SelectError):
        select("transpose", {"perm": (2, 1, 0)})
    assert select("matmul_epilogue", {"act": "none"})[0] == "matmul_epilogue"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "fp16", "fp32"])[0] == "matmul_epilogue_f16w"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "q4_0", "fp32"])[0] == "matmul_epilogue"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "q4_0", "fp32"],
                  "q4_0_kgroup")[0] == "matmul_epilogue_q4k"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "q4_0", "fp32", "fp16"])[0] == "matmul_epilogue_res"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "q4_0", "fp32", "fp16"],
                  "q4_0_kgroup")[0] == "matmul_epilogue_q4k_res"
    assert select("matmul_epilogue", {"act": "none"}, ["fp16", "q8_0", "fp32", "fp16"])[0] == "matmul_epilogue_q8k_res"
    with pytest.raises(SelectError):
        select("softmax", {"axis": 0})


def test_fuse_folds_bias_and_gelu_but_not_residuals():
    t = {n: Tensor(n, "fp32", s, c) for n, s, c in [
        ("x", (4, 8), False), ("w", (8, 8), True), ("b", (8,), True), ("mm", (4, 8), False),
        ("y", (4, 8), False), ("g", (4, 8), False), ("r", (4, 8), False)]}
    ops = (Op(0, "matmul", ("x", "w"), ("mm",)), Op(1, "add", ("b", "mm"), ("y",)),
           Op(2, "gelu_erf", ("y",), ("g",)), Op(3, "add", ("x", "g"), ("r",)))
    f = fuse(Graph(t, ops, ("x",), ("r",)))
    assert [op.kind for op in f.ops] == ["matmul_epilogue", "add"]
    assert f.ops[0].attrs["act"] == "gelu_erf" and f.ops[0].inputs == ("x", "w", "b")


def test_batched_graph_shapes():
    from dataclasses import replace
    cfg = replace(E.TINY_ENCODER, batch=3)
    g = fuse(E.build_vision_encoder(cfg))
    assert g.tensor("image").shape == (9, 1, 64, 64)
    assert g.tensor(g.outputs[0]).shape == (3 * 16 // 4, 64)
    kinds = collections.Counter(op.kind for op in g.ops)
    assert kinds["transpose"] == cfg.depth * 5


@pytest.mark.parametrize("cfg", [E.TINY_ENCODER, E.QWEN35_VISION_FP16])
def test_whole_plan_arena_invariants(cfg):
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg)
    wb = WP.build_whole_plan_batch(g, feeds, reuse=False)
    own = [p for p in wb.placements.values() if p.region != "reshape-alias"]
    spans = sorted((p.offset, p.offset + p.nbytes, p.name) for p in own)
    for (a0, a1, an), (b0, b1, bn) in zip(spans, spans[1:]):
        assert a1 <= b0, f"{an} overlaps {bn}"
    assert all(p.offset % WP.ALIGN == 0 for p in own)
    assert spans[-1][1] <= wb.arena_bytes
    f = fuse(g)
    for op in f.ops:
        if op.kind == "reshape":
            assert wb.placements[op.outputs[0]].offset == wb.placements[op.inputs[0]].offset
    assert wb.placements["pos_embed"].dtype == "fp16"
    assert wb.n_ops + wb.skipped_reshapes == len(f.ops)


@pytest.mark.parametrize("which", ["tiny", "qwen_b32"])
def test_reused_arena_never_overlaps_live_tensors(which):
    """Two activations may share bytes only if no op step sees both alive
    (lifetimes over reshape-unified owners, inclusive)."""
    from dataclasses import replace
    cfg = E.TINY_ENCODER if which == "tiny" else replace(E.QWEN35_VISION_FP16, batch=32)
    g = E.build_vision_encoder(cfg)
    f = fuse(g)
    feeds = {n: np.zeros(t.shape, np.float32) for n, t in f.tensors.items()
             if t.const or n in f.inputs}
    wb = WP.build_whole_plan_batch(g, feeds)
    pl = wb.placements
    own = {n for n, p in pl.items() if p.region == "act"}
    alias = {}
    for op in f.ops:
        if op.kind == "reshape":
            alias[op.outputs[0]] = op.inputs[0]

    def owner(n):
        while n in alias:
            n = alias[n]
        return n
    life = {}
    for i, op in enumerate(f.ops):
        for n in op.inputs + op.outputs:
            o = owner(n)
            if o in own:
                a, b = life.get(o, (i, i))
                life[o] = (min(a, i), max(b, i))
    names = sorted(own)
    for i, a in enumerate(names):
        pa = pl[a]
        for b in names[i + 1:]:
            pb = pl[b]
            if pa.offset < pb.offset + pb.nbytes and pb.offset < pa.offset + pa.nbytes:
                (fa, la), (fb, lb) = life[a], life[b]
                assert la < fb or lb < fa, f"{a} and {b} share bytes while both live"
    assert wb.arena_bytes < 2 ** 32


def test_whole_plan_q4_layouts():
    from dataclasses import replace
    cfg = replace(E.TINY_ENCODER, weight_dtype="q4_0", norm="layernorm")
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg)
    a = WP.build_whole_plan_batch(g, feeds)
    b = WP.build_whole_plan_batch(g, feeds, weight_layout="q4_0_kgroup")
    assert set(a.op_specs) >= {"matmul_epilogue"} and "matmul_epilogue_q4k" not in a.op_specs
    assert "matmul_epilogue_q4k" in b.op_specs
    assert b.placements["blk0.wq"].layout == "q4_0_kgroup"
    assert a.placements["blk0.wq"].nbytes == 64 * 64 // 32 * 18


def test_a_spec_refuses_the_wrong_rank():
    """`ne` is padded to four, so softmax's rows:0:2 / dim:0:2 read a rank-2
    input as C = 1 -- a correctly-shaped wrong answer. The host refuses it."""
    from hexlib_amd.exec.runner import SPECS
    SPECS["softmax"].check_rank([(12, 256, 256)])
    with pytest.raises(ValueError, match="rank-3"):
        SPECS["softmax"].check_rank([(6, 256)])
    with pytest.raises(ValueError, match="rank-2"):
        SPECS["layernorm"].check_rank([(2, 256, 768)])
    SPECS["add"].check_rank([(5,)])


def test_fused_attention_plan():
    """attention="fused": one attention op per block replaces the eight ops
    of the reference chain (3 head transposes, scale, transpose_hd, 2 matmuls,
    softmax, output transpose -> 9 ops, minus the new one)."""
    from dataclasses import replace as _replace
    from hexlib_amd.exec.runner import KIND_ID
    for cfg in (_replace(E.QWEN35_VISION_FP16, attention="fused"),
                _replace(E.QWEN35_VISION_FP16, attention="fused", batch=2)):
        g = E.build_vision_encoder(cfg)
        wb = WP.build_whole_plan_batch(g, E.synthetic_feeds(g, cfg))
        assert wb.n_ops == 259 - 12 * 8
        assert sum(1 for s in wb.op_specs if s == "attention") == 12
        assert KIND_ID["attention"] == 18
    for cfg in (_replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope"),
                _replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope", batch=2)):
        g = E.build_vision_encoder(cfg)
        wb = WP.build_whole_plan_batch(g, E.synthetic_feeds(g, cfg))
        assert wb.n_ops == 259 - 12 * 11       # two fewer linears, one rope op instead of two
        assert sum(1 for s in wb.op_specs if s == "attention_qk_v") == 12
        assert sum(1 for s in wb.op_specs if s == "rope_2d_qk") == 12
        assert not any(s == "rope_2d" for s in wb.op_specs)
        assert KIND_ID["attention_qk_v"] == 19 and KIND_ID["rope_2d_qk"] == 20


def test_fused_qkv_feeds_compute_the_reference_function():
    """fuse_qkv_feeds only rearranges values: on the oracle, the fused-QKV
    graph gives the reference graph's output."""
    from dataclasses import replace as _replace
    from oracle import eager
    cfg = E.TINY_ENCODER
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=3)
    gq = E.build_vision_encoder(_replace(cfg, attention="fused_qkv_rope"))
    want = eager.run_fp32(fuse(g), feeds)[g.outputs[0]]
    got = eager.run_fp32(fuse(gq), E.fuse_qkv_feeds(feeds, cfg))[gq.outputs[0]]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_fuse_residual():
    """Each block's two residual adds fold into the fp16 linear feeding them,
    and so does the pos_embed add (a stored table of the output's shape) into
    the patch-embed linear; q4_0 linears do not; on the storage-rounding
    oracle the result is unchanged bit for bit."""
    from dataclasses import replace as _replace
    from hexlib_amd.graph.fuse import fuse_residual
    from oracle import eager
    cfg = E.TINY_ENCODER
    g = E.build_vision_encoder(cfg)
    f = fuse(g)
    r = fuse_residual(f)
    assert len(f.ops) - len(r.ops) == 2 * cfg.depth + 1
    assert sum(1 for o in r.ops if o.kind == "matmul_epilogue" and len(o.inputs) == 4) == 2 * cfg.depth + 1
    assert sum(1 for o in r.ops if o.kind == "add") == 0
    feeds = E.synthetic_feeds(g, cfg, seed=5)
    a = eager.run_stored(f, feeds)[g.outputs[0]]
    b = eager.run_stored(r, feeds)[g.outputs[0]]
    np.testing.assert_array_equal(a, b)
    # quantized weights fold in any layout; fp16 ones only when their layout allows
    q4 = fuse(E.build_vision_encoder(_replace(E.TINY_ENCODER, weight_dtype="q4_0")))
    rq = fuse_residual(q4, fp16_weights=False)
    assert len(q4.ops) - len(rq.ops) == 2 * cfg.depth + 1
    assert fuse_residual(f, fp16_weights=False) is f
    wbq = WP.build_whole_plan_batch(q4, E.synthetic_feeds(q4, _replace(E.TINY_ENCODER, weight_dtype="q4_0")),
                                    fuse_first=False, weight_layout=None, residual=True)
    assert sum(1 for s in wbq.op_specs if s == "matmul_epilogue_res") == 2 * cfg.depth + 1
    cfgq = _replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    gq = E.build_vision_encoder(cfgq)
    wb = WP.build_whole_plan_batch(gq, E.synthetic_feeds(gq, cfgq), residual=True)
    assert wb.n_ops == 259 - 12 * 11 - 25
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_f16wt_res") == 25


def test_fuse_rope():
    """The q/k rope of each block folds into its fused q/k/v linear and the
    attention reads q, k, v from the linear's output; on the storage-rounding
    oracle the encoder output is unchanged bit for bit. Only the fused-QKV
    graph form has the pattern."""
    from dataclasses import replace as _replace
    from hexlib_amd.graph.fuse import fuse_rope
    from oracle import eager
    cfg = _replace(E.TINY_ENCODER, attention="fused_qkv_rope")
    g = E.build_vision_encoder(cfg)
    f = fuse(g)
    r = fuse_rope(f)
    assert len(f.ops) - len(r.ops) == cfg.depth
    assert not any(o.kind == "rope_2d_qk" for o in r.ops)
    assert sum(1 for o in r.ops if o.kind == "matmul_epilogue" and len(o.inputs) == 5) == cfg.depth
    assert sum(1 for o in r.ops if o.kind == "attention" and len(o.inputs) == 1) == cfg.depth
    feeds = E.fuse_qkv_feeds(E.synthetic_feeds(E.build_vision_encoder(E.TINY_ENCODER), E.TINY_ENCODER,
                                               seed=6), cfg)
    a = eager.run_stored(f, feeds)[g.outputs[0]]
    b = eager.run_stored(r, feeds)[g.outputs[0]]
    np.testing.assert_array_equal(a, b)
    for other in ("unfused", "fused"):
        fo = fuse(E.build_vision_encoder(_replace(E.TINY_ENCODER, attention=other)))
        assert fuse_rope(fo) is fo
    cfgq = _replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    gq = E.build_vision_encoder(cfgq)
    wb = WP.build_whole_plan_batch(gq, E.synthetic_feeds(gq, cfgq), residual=True, rope=True)
    assert wb.n_ops == 259 - 12 * 11 - 25 - 12
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_f16wt_rope") == 12
    assert sum(1 for s in wb.op_specs if s == "attention_qkv") == 12
    assert KIND_ID_OF("matmul_epilogue_f16wt_rope") == 22 and KIND_ID_OF("attention_qkv") == 23
    # rope needs the transposed fp16 weight layout: with another one nothing folds
    wb2 = WP.build_whole_plan_batch(gq, E.synthetic_feeds(gq, cfgq), weight_layout=None, rope=True)
    assert wb2.n_ops == 259 - 12 * 11


def KIND_ID_OF(name):
    from hexlib_amd.exec.runner import KIND_ID
    return KIND_ID[name]


def test_fuse_layernorm():
    """Each block's LN2 folds into fc1, the linear it feeds. LN1 feeds the
    q/k/v linear whose rope tables would give the fused op seven sources, one
    more than a wire op carries, so it stays; so does the final LayerNorm,
    which feeds the merger's reshape. On the storage-rounding oracle the output
    is unchanged bit for bit. Feature counts outside 512..768, more rows than
    the limit, and q4_0 weights do not fold."""
    from dataclasses import replace as _replace
    from hexlib_amd.graph.fuse import fuse_layernorm, fuse_residual, fuse_rope
    from oracle import eager
    cfg = _replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    g = E.build_vision_encoder(cfg)
    f = fuse_residual(fuse_rope(fuse(g)))
    r = fuse_layernorm(f)
    assert len(f.ops) - len(r.ops) == cfg.depth
    assert sum(1 for o in r.ops if o.kind == "layernorm") == cfg.depth + 1
    assert sum(1 for o in r.ops if o.kind == "layernorm_matmul_epilogue") == cfg.depth
    feeds = E.synthetic_feeds(g, cfg, seed=8)
    np.testing.assert_array_equal(eager.run_stored(f, feeds)[g.outputs[0]],
                                  eager.run_stored(r, feeds)[g.outputs[0]])
    assert fuse_layernorm(f, max_rows=255) is f
    tiny = fuse(E.build_vision_encoder(E.TINY_ENCODER))
    assert fuse_layernorm(tiny) is tiny                     # hidden size below 512
    q4 = fuse(E.build_vision_encoder(_replace(E.QWEN35_VISION_FP16, weight_dtype="q4_0")))
    assert fuse_layernorm(q4) is q4
    wb = WP.build_whole_plan_batch(g, E.synthetic_feeds(g, cfg), residual=True, rope=True, layernorm=True)
    assert wb.n_ops == 259 - 12 * 11 - 25 - 12 - 12
    assert sum(1 for s in wb.op_specs if s == "layernorm_matmul_epilogue_f16wt") == 12
    assert KIND_ID_OF("layernorm_matmul_epilogue_f16wt") == 24


def test_problems_names_every_structural_defect():
    """Each defect the reference validator rejects (`hexlib/graph/ir.py:175-225`)
    is reported, and a well-formed graph reports none."""
    from hexlib_amd.graph.ir import Graph, Op, Tensor

    def T(n, const=False):
        return Tensor(n, "fp16", (4,), const)

    ok = Graph({n: T(n) for n in "xyz"} | {"w": T("w", True)},
               (Op(0, "add", ("x", "w"), ("y",)), Op(1, "scale", ("y",), ("z",))), ("x",), ("z",))
    assert ok.problems() == []

    def probs(ops, inputs=("x",), outputs=("z",), extra=()):
        tens = {n: T(n) for n in "xyz"} | {"w": T("w", True)} | {t.name: t for t in extra}
        return " | ".join(Graph(tens, tuple(ops), inputs, outputs).problems())

    assert "no ops" in probs([], outputs=("x",))
    assert "nothing marked as an output" in probs([Op(0, "scale", ("x",), ("z",))], outputs=())
    assert "share id 0" in probs([Op(0, "scale", ("x",), ("y",)), Op(0, "scale", ("y",), ("z",))])
    assert "input 'q' not in the tensor table" in probs([Op(0, "add", ("x", "q"), ("z",))])
    assert "output 'q' not in the tensor table" in probs([Op(0, "scale", ("x",), ("q",)),
                                                           Op(1, "scale", ("x",), ("z",))])
    assert "input 'y' has no producer" in probs([Op(0, "add", ("x", "y"), ("z",))])
    assert "produced later" in probs([Op(0, "scale", ("y",), ("z",)), Op(1, "scale", ("x",), ("y",))])
    assert "already produced by scale #0" in probs([Op(0, "scale", ("x",), ("z",)),
                                                    Op(1, "scale", ("x",), ("z",))])
    assert "already produced by a graph input" in probs([Op(0, "scale", ("w",), ("x",)),
                                                         Op(1, "scale", ("x",), ("z",))])
    assert "output 'z': no op produces it" in probs([Op(0, "scale", ("x",), ("y",))])
    assert "input 'q': not in the tensor table" in probs([Op(0, "scale", ("x",), ("z",))],
                                                          inputs=("x", "q"))
