"""Whole-plan parity on the GPU: one blob, one arena, every op through the
dispatcher and the generated entries, eager and as one captured hipGraph.

Compared with the oracle's storage-rounding executor (`oracle.eager.run_stored`,
the reference `interpreter.run` numerics) on the same seeded feeds; BASELINE's
whole-encoder bar is 2e-2 max abs. Graph replays are checked against the eager
run bit for bit, several times over with eager work in between.
"""
from dataclasses import replace

import numpy as np
import pytest

from hexlib_amd import encoder as E
from hexlib_amd.exec.gpu import GpuBackend, GpuPlan, GpuSession
from hexlib_amd.exec.wholeplan import build_whole_plan_batch
from hexlib_amd.graph.fuse import fuse
from oracle import eager
from oracle.quant import dequantize_q4_0_fp16
from hexlib_amd.quant import pack_q4_0_kgrouped, pack_q4_0_nblocked

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def session(torch_gpu):
    s = GpuSession()
    yield s
    s.close()


def _run_plan(session, cfg, feeds, graph_mode, weight_layout=None, repeats=1, residual=False, rope=False,
              layernorm=False, fold_ln_rows=0):
    g = E.build_vision_encoder(cfg)
    wb = build_whole_plan_batch(g, feeds, weight_layout=weight_layout, residual=residual, rope=rope,
                                layernorm=layernorm, fold_ln_rows=fold_ln_rows)
    plan = GpuPlan(wb, session)
    try:
        outs = []
        for _ in range(repeats):
            rsp = plan.run(graph=graph_mode)
            assert rsp.ok and rsp.n_ops == wb.n_ops
            outs.append(plan.read(g.outputs[0]))
        return outs, wb
    finally:
        plan.close()


def _oracle(cfg, feeds, dense_weights=None):
    g = fuse(E.build_vision_encoder(cfg))
    f = dict(feeds)
    if dense_weights:
        f.update(dense_weights)
    return eager.run_stored(g, f)[g.outputs[0]]


@pytest.mark.parametrize("cfg", [E.TINY_ENCODER, replace(E.TINY_ENCODER, norm="layernorm"),
                                 replace(E.TINY_ENCODER, attention="fused"),
                                 replace(E.TINY_ENCODER, attention="fused_qkv_rope")])
def test_tiny_encoder_eager_and_graph(session, cfg):
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=0)
    want = _oracle(cfg, feeds)
    (eager_out,), _ = _run_plan(session, cfg, feeds, graph_mode=False)
    graph_outs, _ = _run_plan(session, cfg, feeds, graph_mode=True, repeats=3)
    err = np.abs(eager_out - want).max()
    print(f"[tiny {cfg.norm}] max abs vs oracle {err:.3e}", flush=True)
    assert err <= 2e-2
    for o in graph_outs:
        np.testing.assert_array_equal(o, eager_out)


def test_golden_config_fp16_on_gpu(session, golden):
    cfg = replace(E.GOLDEN_TINY, act_dtype="fp16", weight_dtype="fp16")
    g = E.build_vision_encoder(cfg)
    feeds = E.feeds_from_params(g, cfg, lambda n: golden["param::" + n])
    feeds = {k: (v.astype(np.float16).astype(np.float32) if g.tensor(k).dtype == "fp16" else v)
             for k, v in feeds.items()}
    feeds["image"] = golden["image"]
    (out,), _ = _run_plan(session, cfg, feeds, graph_mode=True)
    want = _oracle(cfg, feeds)
    up = golden["expected_merged"]
    print(f"[golden fp16] vs oracle {np.abs(out - want).max():.3e} vs upstream {np.abs(out - up).max():.3e}",
          flush=True)
    assert np.abs(out - want).max() <= 2e-2
    assert np.abs(out - up).max() <= 2e-2


def test_qwen_encoder_256_fp16(session):
    cfg = E.QWEN35_VISION_FP16
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=0)
    (out,), wb = _run_plan(session, cfg, feeds, graph_mode=True)
    assert wb.n_ops == 259
    want = _oracle(cfg, feeds)
    err = np.abs(out - want).max()
    print(f"[qwen 256 fp16] max abs {err:.3e} (|out| max {np.abs(want).max():.3f})", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("layout,residual", [(None, False), ("q4_0_kgroup", False), (None, True),
                                             ("q4_0_kgroup", True)])
def test_qwen_encoder_reference_q4_config(session, layout, residual):
    """The reference's own shipped config: T=2, q4_0 weights. The oracle gets
    the dequantized, fp16-rounded weights the kernel multiplies with. With
    `residual` the residual adds ride in the q4_0 linears' epilogues (KIND 28
    blocked along N, KIND 30 grouped along K)."""
    cfg = replace(E.QWEN35_VISION_Q4, depth=2)
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=1)
    dense = {}
    for t in g.tensors.values():
        if t.dtype == "q4_0":
            w = feeds[t.name]
            if layout == "q4_0_kgroup":
                dq = dequantize_q4_0_fp16(pack_q4_0_kgrouped(w), w.shape[::-1]).T
            else:
                dq = dequantize_q4_0_fp16(pack_q4_0_nblocked(w), w.shape)
            dense[t.name] = np.ascontiguousarray(dq)
    (out,), wb = _run_plan(session, cfg, feeds, graph_mode=True, weight_layout=layout, residual=residual)
    if residual:
        res_spec = "matmul_epilogue_q4k_res" if layout == "q4_0_kgroup" else "matmul_epilogue_res"
        assert sum(1 for s in wb.op_specs if s == res_spec) == 2 * cfg.depth + 1
    want = _oracle(cfg, feeds, dense)
    err = np.abs(out - want).max()
    print(f"[qwen q4 {layout} residual={residual}] max abs {err:.3e}", flush=True)
    assert err <= 2e-2


def test_qwen_encoder_q8_0_fused(session):
    """The bench's q8_0 plan: fused q/k/v with the q/k rope in the q8_0 GEMM's
    epilogue (KIND 31, attention reading its output), the residual adds in
    the q8_0 linears' epilogues (KIND 29): against the storage-rounding oracle
    of the REFERENCE graph on the dequantized weights, <= 2e-2 max abs."""
    from hexlib_amd.quant import pack_q8_0_kgrouped
    from oracle.quant import dequantize_q8_0_fp16
    cfg_ref = replace(E.QWEN35_VISION_Q8, depth=4)
    g_ref = E.build_vision_encoder(cfg_ref)
    feeds = E.synthetic_feeds(g_ref, cfg_ref, seed=2)
    dense = {}
    for t in g_ref.tensors.values():
        if t.dtype == "q8_0":
            w = feeds[t.name]
            dense[t.name] = np.ascontiguousarray(dequantize_q8_0_fp16(pack_q8_0_kgrouped(w), w.shape[::-1]).T)
    cfg = replace(cfg_ref, attention="fused_qkv_rope")
    (out,), wb = _run_plan(session, cfg, E.fuse_qkv_feeds(feeds, cfg), graph_mode=True, weight_layout="auto",
                           residual=True, rope=True)
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_q8k_rope") == cfg.depth
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_q8k_res") == 2 * cfg.depth + 1
    want = _oracle(cfg_ref, feeds, dense)
    err = np.abs(out - want).max()
    print(f"[qwen q8_0 fused] max abs vs reference graph {err:.3e}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("residual", [False, True])
def test_qwen_encoder_q8_0(session, residual):
    """cfg 4 with q8_0 weights (KIND 25 for every linear; with `residual`
    KIND 29 for the two residual linears of each block and the patch embed).
    The oracle gets the dequantized, fp16-rounded weights the kernel
    multiplies with; the output also stays close to the fp16-weight encoder's
    (cosine > 0.999)."""
    from hexlib_amd.quant import pack_q8_0_kgrouped
    from oracle.quant import dequantize_q8_0_fp16
    cfg = replace(E.QWEN35_VISION_Q8, depth=4)
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=1)
    dense = {}
    for t in g.tensors.values():
        if t.dtype == "q8_0":
            w = feeds[t.name]
            dense[t.name] = np.ascontiguousarray(dequantize_q8_0_fp16(pack_q8_0_kgrouped(w), w.shape[::-1]).T)
    (out,), wb = _run_plan(session, cfg, feeds, graph_mode=True, weight_layout="auto" if residual else None,
                           residual=residual)
    n_res = 2 * cfg.depth + 1 if residual else 0
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_q8k") == 6 * cfg.depth + 3 - n_res
    assert sum(1 for s in wb.op_specs if s == "matmul_epilogue_q8k_res") == n_res
    want = _oracle(cfg, feeds, dense)
    err = np.abs(out - want).max()
    cfg16 = replace(cfg, weight_dtype="fp16")
    (ref16,), _ = _run_plan(session, cfg16, feeds, graph_mode=True)
    cos = float(np.dot(out.ravel(), ref16.ravel()) / (np.linalg.norm(out) * np.linalg.norm(ref16)))
    print(f"[qwen q8_0] max abs vs oracle {err:.3e}; cosine vs fp16 weights {cos:.6f}", flush=True)
    assert err <= 2e-2
    assert cos > 0.999


def test_batched_encoder_matches_per_image(session):
    cfg1 = E.TINY_ENCODER
    cfgb = replace(cfg1, batch=3)
    gb = E.build_vision_encoder(cfgb)
    feeds_b = E.synthetic_feeds(gb, cfgb, seed=2)
    (out_b,), _ = _run_plan(session, cfgb, feeds_b, graph_mode=True)
    g1 = E.build_vision_encoder(cfg1)
    per = out_b.shape[0] // 3
    for i in range(3):
        f1 = {}
        for t in g1.tensors.values():
            if t.name == "image":
                f1["image"] = feeds_b["image"][i * 3:(i + 1) * 3]
            elif t.name in ("pos_embed", "rope_cos", "rope_sin"):
                n = cfg1.num_tokens
                f1[t.name] = feeds_b[t.name][i * n:(i + 1) * n]
            elif t.const:
                f1[t.name] = feeds_b[t.name]
        want = _oracle(cfg1, f1)
        assert np.abs(out_b[i * per:(i + 1) * per] - want).max() <= 2e-2


def test_per_op_backend_through_the_wire(session):
    be = GpuBackend(session)
    r = np.random.default_rng(3)
    x = r.standard_normal((12, 256, 64)).astype(np.float16)
    y, rsp = be.run("transpose", [x], {"perm": (0, 2, 1)}, (12, 64, 256))
    np.testing.assert_array_equal(y, np.transpose(x, (0, 2, 1)))
    assert rsp.results[0].cycles > 0                      # timed: GPU ns
    s = (r.standard_normal((12, 256, 256)) * 0.125).astype(np.float16)
    y, _ = be.run("softmax", [s], {"axis": -1}, s.shape)
    xs = s.astype(np.float64)
    want = np.exp(xs - xs.max(-1, keepdims=True))
    want /= want.sum(-1, keepdims=True)
    assert np.abs(y.astype(np.float64) - want).max() <= 2e-3
    a = r.standard_normal((64, 128)).astype(np.float16)
    w = (r.standard_normal((128, 96)) * 0.05).astype(np.float32)
    b = np.zeros(96, np.float32)
    y, _ = be.run("matmul_epilogue", [a, w, b], {"act": "gelu_tanh"}, (64, 96))
    from oracle import kernels as K
    want = K.matmul_epilogue_fp16(a, pack_q4_0_nblocked(w), b, 128, 96, 1)
    assert K.close_f16(y, want, 0.01, 3e-4).all()


def test_interpreter_backends_every_kind(session):
    """The reference-shaped adapter (`interpreter_backends(gpu)[kind](arrays,
    attrs) -> (out,)`, as `hexlib/exec/dsp.py:656-715` hands to the plan
    executor) for every kernel kind, fed fp32 arrays like the executor's
    compute dtype, against the op registry reference on the fp16-rounded
    inputs the wire carries."""
    from hexlib_amd import encoder as E
    from hexlib_amd.exec.gpu import interpreter_backends
    from oracle import kernels as K
    from oracle.refs import REFERENCES
    be = interpreter_backends(GpuBackend(session))
    r = np.random.default_rng(5)

    def f(*s):
        return r.standard_normal(s).astype(np.float32)

    def r16(a):
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)

    cos, sin = E.rope_tables(E.TINY_ENCODER)
    T = cos.shape[0]
    cases = [
        ("add", [f(64, 96), f(64, 96)], {}, [True, True]),
        ("scale", [f(12, 64, 32)], {"factor": 0.125}, [True]),
        ("cast", [f(64, 96)], {"dtype": "fp16"}, [False]),
        ("softmax", [f(2, 6, 256)], {"axis": -1}, [True]),
        ("layernorm", [f(16, 768), 1 + 0.02 * f(768), 0.02 * f(768)], {"eps": 1e-6}, [True, False, False]),
        ("rmsnorm", [f(16, 768), 1 + 0.02 * f(768)], {"eps": 1e-6}, [True, True]),
        ("rope_2d", [f(T, 2, cos.shape[1]), cos, sin], {}, [True, False, False]),
        ("transpose", [f(16, 3, 64)], {"perm": (1, 0, 2)}, [True]),
        ("transpose", [f(6, 40, 24)], {"perm": (0, 2, 1)}, [True]),
        ("patchify", [r.random((3, 1, 64, 64), dtype=np.float32)],
         {"patch": 16, "temporal_patch": 1, "merge": 2, "grid_h": 4, "grid_w": 4}, [False]),
        ("matmul", [f(3, 40, 64), 0.1 * f(3, 64, 48)], {}, [True, True]),
    ]
    for kind, arrays, attrs, rounded in cases:
        (got,) = be[kind](arrays, attrs)
        ins = [r16(a) if rd else a for a, rd in zip(arrays, rounded)]
        (want,) = REFERENCES[kind](ins, attrs)
        want = np.asarray(want, np.float32)
        exact = kind in ("transpose", "patchify", "cast")
        if exact:
            np.testing.assert_array_equal(np.asarray(got, np.float32), want.astype(got.dtype).astype(np.float32))
        else:
            assert K.close_f16(got, want.astype(np.float16), 0.02, 2e-3).all(), kind
    # matmul_epilogue: the dense weight is quantized to q4_0 on the way in
    a, w, b = f(32, 128), 0.05 * f(128, 64), 0.02 * f(64)
    (got,) = be["matmul_epilogue"]([a, w, b], {"act": "gelu_tanh"})
    want = K.matmul_epilogue_fp16(a.astype(np.float16), pack_q4_0_nblocked(w), b, 128, 64, 1)
    assert K.close_f16(got, want, 0.01, 3e-4).all()


@pytest.mark.parametrize("image,batch,mode,residual,rope,ln", [
    (256, 1, "fused", False, False, False), (448, 1, "fused", False, False, False),
    (256, 4, "fused", False, False, False),
    (256, 1, "fused_qkv_rope", False, False, False), (448, 1, "fused_qkv_rope", False, False, False),
    (256, 4, "fused_qkv_rope", False, False, False),
    (256, 1, "fused_qkv_rope", True, False, False), (448, 1, "fused_qkv_rope", True, False, False),
    (256, 4, "fused_qkv_rope", True, False, False),
    (256, 1, "fused_qkv_rope", True, True, False), (448, 1, "fused_qkv_rope", True, True, False),
    (256, 4, "fused_qkv_rope", True, True, False), (256, 1, "fused_qkv_rope", False, True, False),
    (256, 1, "fused_qkv_rope", True, True, True), (448, 1, "fused_qkv_rope", True, True, True),
    (256, 4, "fused_qkv_rope", True, True, True), (256, 1, "fused", False, False, True)])
def test_fused_attention_encoder_matches_the_reference_graph(session, image, batch, mode, residual, rope, ln):
    """The plan with one fused attention op per block (and, with `residual`
    / `rope` / `ln`, those folded into the linears) against the storage-
    rounding oracle of the REFERENCE graph (unfused attention chain): the
    whole-encoder bar, <= 2e-2 max abs."""
    base = E.QWEN35_VISION_FP16 if image == 256 else E.encoder_at(image)
    cfg_ref = replace(base, batch=batch)
    g_ref = E.build_vision_encoder(cfg_ref)
    feeds = E.synthetic_feeds(g_ref, cfg_ref, seed=4)
    cfg = replace(cfg_ref, attention=mode)
    fused_feeds = E.fuse_qkv_feeds(feeds, cfg) if mode == "fused_qkv_rope" else feeds
    (out,), wb = _run_plan(session, cfg, fused_feeds, graph_mode=True, residual=residual, rope=rope,
                           layernorm=ln, weight_layout="auto" if residual or rope or ln else None)
    assert wb.n_ops == (259 - 12 * (8 if mode == "fused" else 11) - (25 if residual else 0)
                        - (12 if rope else 0) - (12 if ln else 0))
    want = _oracle(cfg_ref, feeds)
    err = np.abs(out - want).max()
    print(f"[{mode} residual={residual} rope={rope} ln={ln} {image} b{batch}] max abs vs reference graph "
          f"{err:.3e}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("image,batch", [(256, 1), (256, 4), (448, 1)])
def test_folded_layernorm_plan_matches_the_reference_graph(session, image, batch):
    """The bench's batch-1 product plan -- fused q/k/v + rope, fused
    attention, residual epilogues, and every block LayerNorm folded into the
    linear it feeds (66 launches at batch 1) -- here also at batch 4 and at
    448x448 with the fold allowed at those row counts: against the storage-
    rounding oracle of the REFERENCE graph, <= 2e-2 max abs; graph replays
    equal to each other bit for bit."""
    base = E.QWEN35_VISION_FP16 if image == 256 else E.encoder_at(image)
    cfg_ref = replace(base, batch=batch)
    g_ref = E.build_vision_encoder(cfg_ref)
    feeds = E.synthetic_feeds(g_ref, cfg_ref, seed=5)
    cfg = replace(cfg_ref, attention="fused_qkv_rope")
    outs, wb = _run_plan(session, cfg, E.fuse_qkv_feeds(feeds, cfg), graph_mode=True, repeats=3, residual=True,
                         rope=True, weight_layout="auto", fold_ln_rows=cfg.num_tokens * batch)
    assert wb.n_ops == 259 - 12 * 11 - 25 - 12 - 24
    assert sum(s.startswith("lnfold_matmul_epilogue") for s in wb.op_specs) == 24
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    want = _oracle(cfg_ref, feeds)
    err = np.abs(outs[0] - want).max()
    print(f"[folded layernorm {image} b{batch}] max abs vs reference graph {err:.3e}", flush=True)
    assert err <= 2e-2


def test_folded_layernorm_product_plan_at_batch_32(session):
    """The batch-32 product plan with every block LayerNorm folded into the
    linear it feeds (the large-tile form's KIND 26 / 27): images 0 and 31
    against the storage-rounding oracle of the REFERENCE graph at batch 1 on
    that image's feeds, <= 2e-2 max abs."""
    cfg1 = E.QWEN35_VISION_FP16
    cfg_ref = replace(cfg1, batch=32)
    g_ref = E.build_vision_encoder(cfg_ref)
    feeds = E.synthetic_feeds(g_ref, cfg_ref, seed=7)
    cfg = replace(cfg_ref, attention="fused_qkv_rope")
    (out,), wb = _run_plan(session, cfg, E.fuse_qkv_feeds(feeds, cfg), graph_mode=True, residual=True,
                           rope=True, weight_layout="auto", fold_ln_rows=32 * cfg1.num_tokens)
    assert wb.n_ops == 259 - 12 * 11 - 25 - 12 - 24
    per = out.shape[0] // 32
    for i in (0, 31):
        want = _oracle(cfg1, _image_feeds(cfg1, feeds, i))
        err = np.abs(out[i * per:(i + 1) * per] - want).max()
        print(f"[folded layernorm b32] image {i}: max abs vs reference graph {err:.3e}", flush=True)
        assert err <= 2e-2


def _image_feeds(cfg1, feeds_b, i):
    """Image i's feeds at batch 1, sliced from a batch's feeds: its channels of
    the stacked image, its rows of the per-token tables, every const shared."""
    g1 = E.build_vision_encoder(cfg1)
    n = cfg1.num_tokens
    c = cfg1.in_channels
    f1 = {}
    for t in g1.tensors.values():
        if t.name == "image":
            f1["image"] = feeds_b["image"][i * c:(i + 1) * c]
        elif t.name in ("pos_embed", "rope_cos", "rope_sin"):
            f1[t.name] = feeds_b[t.name][i * n:(i + 1) * n]
        elif t.const:
            f1[t.name] = feeds_b[t.name]
    return f1


def test_product_plan_at_batch_32(session):
    """BASELINE cfg 4 at batch 32 (M = 8192 for every linear), run as the
    bench's product plan: fused attention over one q/k/v projection with the
    q/k rope in its GEMM epilogue, residual adds in the proj/fc2 epilogues,
    W^T weights. Images 0, 17 and 31 are each checked against the storage-
    rounding oracle of the REFERENCE graph at batch 1 on that image's feeds
    (the reference executor is single-image, `hexlib/exec/interpreter.py:80-205`);
    the whole-encoder bar is 2e-2 max abs."""
    cfg1 = E.QWEN35_VISION_FP16
    cfg_ref = replace(cfg1, batch=32)
    g_ref = E.build_vision_encoder(cfg_ref)
    feeds = E.synthetic_feeds(g_ref, cfg_ref, seed=6)
    cfg = replace(cfg_ref, attention="fused_qkv_rope")
    (out,), wb = _run_plan(session, cfg, E.fuse_qkv_feeds(feeds, cfg), graph_mode=True, residual=True,
                           rope=True, weight_layout="auto")
    assert wb.n_ops == 259 - 12 * 11 - 25 - 12
    per = out.shape[0] // 32
    for i in (0, 17, 31):
        want = _oracle(cfg1, _image_feeds(cfg1, feeds, i))
        err = np.abs(out[i * per:(i + 1) * per] - want).max()
        print(f"[product plan b32] image {i}: max abs vs reference graph {err:.3e}", flush=True)
        assert err <= 2e-2
