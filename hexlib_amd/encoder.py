"""The ViT vision-encoder graph (Qwen3.5 vision tower shape) and its feeds.

Graph structure follows the reference builder op for op
(`hexlib/models/vit.py:113-218`): patchify -> cast -> patch-embed linear ->
+pos_embed -> depth x [norm -> q/k/v linears -> reshape -> rope(q,k) ->
transpose(1,0,2) -> scale(q) -> transpose(0,2,1)(k) -> matmul -> softmax ->
matmul -> transpose back -> reshape -> proj linear -> residual -> norm -> fc1
-> gelu_tanh -> fc2 -> residual] -> merger norm -> reshape -> fc1 -> gelu_erf
-> fc2. At batch 1 with `norm="layernorm"` the fused graph is the reference's
308-step plan (49 reshape, 24 matmul, 75 matmul_epilogue).

Build extensions (not in the reference, each optional and off by default):
* `batch` > 1: a leading image axis. Linears see M = batch * tokens, attention
  runs over batch * heads, the per-token tables are replicated per image.
* `norm="rmsnorm"`: RMSNorm blocks with an fp16 gain and no bias, matching the
  reference's `rmsnorm_fp16` kernel contract.
* `attention="fused"`: each block's attention chain (head transposes, scale,
  transpose_hd, two matmuls, softmax) as one `attention` op; `"fused_qkv_rope"`
  additionally computes q, k, v with one [H, 3H] linear, ropes q and k with one
  `rope_2d_qk` op and reads v from the projection (`fuse_qkv_feeds` rewrites
  reference feeds for it).

Host-side tables (RoPE cos/sin, bilinear pos_embed) restate the reference
loader (`hexlib/models/loader.py:30-146`).
"""
from __future__ import annotations

from dataclasses import dataclass, fields, replace
from typing import Mapping, Any, Callable, get_type_hints

import numpy as np

from hexlib_amd.graph import opdefs  # noqa: F401  (registers op kinds)
from hexlib_amd.graph.ir import Graph, Op, Tensor


@dataclass(frozen=True)
class VitConfig:
    """Reference `hexlib/models/vit.py:18-48`, plus `norm` and `batch`."""

    depth: int
    hidden_size: int
    num_heads: int
    intermediate_size: int
    patch_size: int
    temporal_patch_size: int
    in_channels: int
    spatial_merge_size: int
    out_hidden_size: int
    layernorm_eps: float
    rope_theta: float
    image_size: int
    act_dtype: str = "fp32"
    weight_dtype: str = "fp32"
    norm: str = "layernorm"
    batch: int = 1
    # "unfused": the reference graph; "fused": one attention op per block
    # (KIND 18); "fused_qkv_rope": one q/k/v linear, one rope_2d_qk op on its q
    # and k (KIND 20) and one attention op reading v from it (KIND 19)
    attention: str = "unfused"

    @property
    def grid(self) -> int:
        return self.image_size // self.patch_size

    @property
    def num_tokens(self) -> int:
        return self.grid * self.grid

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def merge_unit(self) -> int:
        return self.spatial_merge_size * self.spatial_merge_size

    @property
    def patch_features(self) -> int:
        return self.in_channels * self.temporal_patch_size * self.patch_size ** 2


# BASELINE cfg 4: the Qwen3.5-0.8B vision tower at 256x256 with fp16 weights
# and activations. temporal_patch_size 1 (single still image, K=768 for the
# patch embedding) where the reference's checkpoint config says 2.
QWEN35_VISION_FP16 = VitConfig(
    depth=12, hidden_size=768, num_heads=12, intermediate_size=3072,
    patch_size=16, temporal_patch_size=1, in_channels=3, spatial_merge_size=2,
    out_hidden_size=1024, layernorm_eps=1e-6, rope_theta=10000.0, image_size=256,
    act_dtype="fp16", weight_dtype="fp16",
)

# The reference's own shipped config (`hexlib/models/qwen35.py:15-42`): T=2,
# q4_0 weights.
QWEN35_VISION_Q4 = replace(QWEN35_VISION_FP16, temporal_patch_size=2, weight_dtype="q4_0")

# q8_0 weights (the reference's README measures q8_0 at cosine 0.999 against
# q4_0's 0.868 on the real model, `README.md:180-191`) on the cfg-4 shape.
QWEN35_VISION_Q8 = replace(QWEN35_VISION_FP16, weight_dtype="q8_0")

# BASELINE cfg 1: the tiny encoder run through the CPU reference executor.
TINY_ENCODER = VitConfig(
    depth=2, hidden_size=64, num_heads=2, intermediate_size=256, patch_size=16,
    temporal_patch_size=1, in_channels=3, spatial_merge_size=2, out_hidden_size=64,
    layernorm_eps=1e-6, rope_theta=10000.0, image_size=64, act_dtype="fp16",
    weight_dtype="fp16", norm="rmsnorm",
)

# The configuration the committed golden vectors were generated at
# (reference `hexlib/tests/test_vision_oracle.py:22-36`).
GOLDEN_TINY = VitConfig(
    depth=2, hidden_size=64, num_heads=4, intermediate_size=128, patch_size=4,
    temporal_patch_size=2, in_channels=3, spatial_merge_size=2, out_hidden_size=32,
    layernorm_eps=1e-6, rope_theta=10000.0, image_size=32,
)


def encoder_at(image_size: int, batch: int = 1, base: VitConfig = QWEN35_VISION_FP16) -> VitConfig:
    return replace(base, image_size=image_size, batch=batch)


class ConfigError(ValueError):
    pass


def config_problems(cfg: VitConfig) -> list[str]:
    """Reference `vit.py:248-283`, plus the extension fields."""
    out: list[str] = []
    hints = get_type_hints(VitConfig)
    for f in fields(VitConfig):
        if hints.get(f.name) is int and getattr(cfg, f.name) <= 0:
            out.append(f"{f.name} {getattr(cfg, f.name)} must be positive")
    if out:
        return out
    if cfg.image_size % cfg.patch_size:
        out.append(f"image_size {cfg.image_size} not divisible by patch_size {cfg.patch_size}")
    elif cfg.grid % cfg.spatial_merge_size:
        out.append(f"patch grid {cfg.grid} not divisible by merge {cfg.spatial_merge_size}")
    if cfg.hidden_size % cfg.num_heads:
        out.append(f"hidden_size {cfg.hidden_size} not divisible by num_heads {cfg.num_heads}")
    elif cfg.head_dim % 2:
        out.append(f"head_dim {cfg.head_dim} must be even for 2D RoPE")
    if cfg.norm not in ("layernorm", "rmsnorm"):
        out.append(f"norm {cfg.norm!r} must be 'layernorm' or 'rmsnorm'")
    if cfg.attention not in ("unfused", "fused", "fused_qkv_rope"):
        out.append(f"attention {cfg.attention!r} must be 'unfused', 'fused' or 'fused_qkv_rope'")
    return out


class _Builder:
    def __init__(self, cfg: VitConfig) -> None:
        self.cfg = cfg
        self.tensors: dict[str, Tensor] = {}
        self.ops: list[Op] = []

    def declare(self, name, shape, dtype, const=False) -> str:
        if name in self.tensors:
            raise ValueError(f"tensor {name!r} declared twice")
        self.tensors[name] = Tensor(name=name, dtype=dtype, shape=tuple(shape), const=const)
        return name

    def const(self, name, shape, dtype=None) -> str:
        return self.declare(name, shape, dtype or self.cfg.weight_dtype, const=True)

    def emit(self, kind, inputs, out, shape, attrs=None, dtype=None) -> str:
        self.declare(out, shape, dtype or self.cfg.act_dtype)
        self.ops.append(Op(id=len(self.ops), kind=kind, inputs=tuple(inputs),
                           outputs=(out,), attrs=attrs or {}))
        return out

    def linear(self, x, wname, bname, k, n, out) -> str:
        w = self.const(wname, (k, n))
        b = self.const(bname, (n,), "fp32")
        rows = self.tensors[x].shape[:-1]
        mm = self.emit("matmul", (x, w), f"{out}.mm", rows + (n,))
        return self.emit("add", (mm, b), out, rows + (n,))

    def norm(self, x, prefix, out) -> str:
        c = self.cfg
        width = self.tensors[x].shape[-1]
        if c.norm == "rmsnorm":
            w = self.const(f"{prefix}_w", (width,), "fp16")
            return self.emit("rmsnorm", (x, w), out, self.tensors[x].shape,
                             {"eps": c.layernorm_eps})
        w = self.const(f"{prefix}_w", (width,), "fp32")
        b = self.const(f"{prefix}_b", (width,), "fp32")
        return self.emit("layernorm", (x, w, b), out, self.tensors[x].shape,
                         {"eps": c.layernorm_eps})


def build_vision_encoder(cfg: VitConfig) -> Graph:
    problems = config_problems(cfg)
    if problems:
        raise ConfigError("invalid vision config: " + "; ".join(problems))
    b = _Builder(cfg)
    B, n, H = cfg.batch, cfg.num_tokens, cfg.hidden_size
    heads, d = cfg.num_heads, cfg.head_dim
    rows = B * n
    feat = cfg.patch_features
    # Batched images are stacked on the channel axis, [B*C, T, H, W], so the
    # image still fits the wire's four extents.
    image = b.declare("image", (B * cfg.in_channels, cfg.temporal_patch_size,
                                cfg.image_size, cfg.image_size), "fp32")
    pattrs = {"patch": cfg.patch_size, "temporal_patch": cfg.temporal_patch_size,
              "merge": cfg.spatial_merge_size, "grid_h": cfg.grid, "grid_w": cfg.grid}
    if B > 1:
        pattrs["batch"] = B
    patches = b.emit("patchify", (image,), "patches", (rows, feat), pattrs, dtype="fp32")
    patches_act = b.emit("cast", (patches,), "patches.cast", (rows, feat),
                         {"dtype": cfg.act_dtype}, dtype=cfg.act_dtype)
    emb = b.linear(patches_act, "w_patch_embed", "b_patch_embed", feat, H, "patch_embed.out")
    pos = b.const("pos_embed", (rows, H), "fp32")
    x = b.emit("add", (emb, pos), "x0", (rows, H))
    cos = b.const("rope_cos", (rows, d), "fp32")
    sin = b.const("rope_sin", (rows, d), "fp32")

    for layer in range(cfg.depth):
        p = f"blk{layer}"
        a = b.norm(x, f"{p}.ln1", f"{p}.ln1.out")
        qkv = {}
        for which in (() if cfg.attention == "fused_qkv_rope" else ("q", "k", "v")):
            proj = b.linear(a, f"{p}.w{which}", f"{p}.b{which}", H, H, f"{p}.{which}.out")
            t = b.emit("reshape", (proj,), f"{p}.{which}.h", (rows, heads, d),
                       {"shape": (rows, heads, d)})
            if which in ("q", "k"):
                t = b.emit("rope_2d", (t, cos, sin), f"{p}.{which}.rope", (rows, heads, d))
            if cfg.attention == "fused":
                qkv[which] = t
                continue
            if B == 1:
                qkv[which] = b.emit("transpose", (t,), f"{p}.{which}.t", (heads, n, d),
                                    {"perm": (1, 0, 2)})
            else:
                t4 = b.emit("reshape", (t,), f"{p}.{which}.b4", (B, n, heads, d),
                            {"shape": (B, n, heads, d)})
                t4 = b.emit("transpose", (t4,), f"{p}.{which}.t4", (B, heads, n, d),
                            {"perm": (0, 2, 1, 3)})
                qkv[which] = b.emit("reshape", (t4,), f"{p}.{which}.t", (B * heads, n, d),
                                    {"shape": (B * heads, n, d)})
        if cfg.attention == "fused_qkv_rope":
            # one [H, 3H] linear for q, k, v; rope_2d and attention in one op
            fused = b.linear(a, f"{p}.wqkv", f"{p}.bqkv", H, 3 * H, f"{p}.qkv.out")
            qkv4 = b.emit("reshape", (fused,), f"{p}.qkv.h", (rows, 3, heads, d),
                          {"shape": (rows, 3, heads, d)})
            qk = b.emit("rope_2d_qk", (qkv4, cos, sin), f"{p}.qk.rope", (rows, 2, heads, d))
            ctxt = b.emit("attention", (qk, qkv4), f"{p}.ctx.t", (rows, heads, d),
                          {"scale": float(d) ** -0.5, "batch": B})
        elif cfg.attention == "fused":
            # one op for the chain below; [rows, heads, d] in and out
            ctxt = b.emit("attention", (qkv["q"], qkv["k"], qkv["v"]), f"{p}.ctx.t", (rows, heads, d),
                          {"scale": float(d) ** -0.5, "batch": B})
        else:
            bh = B * heads
            qs = b.emit("scale", (qkv["q"],), f"{p}.q.scaled", (bh, n, d),
                        {"factor": float(d) ** -0.5})
            ktt = b.emit("transpose", (qkv["k"],), f"{p}.k.tt", (bh, d, n), {"perm": (0, 2, 1)})
            scores = b.emit("matmul", (qs, ktt), f"{p}.scores", (bh, n, n))
            probs = b.emit("softmax", (scores,), f"{p}.probs", (bh, n, n), {"axis": -1})
            ctx = b.emit("matmul", (probs, qkv["v"]), f"{p}.ctx", (bh, n, d))
            if B == 1:
                ctxt = b.emit("transpose", (ctx,), f"{p}.ctx.t", (n, heads, d), {"perm": (1, 0, 2)})
            else:
                c4 = b.emit("reshape", (ctx,), f"{p}.ctx.b4", (B, heads, n, d),
                            {"shape": (B, heads, n, d)})
                ctxt = b.emit("transpose", (c4,), f"{p}.ctx.t", (B, n, heads, d),
                              {"perm": (0, 2, 1, 3)})
        ctxf = b.emit("reshape", (ctxt,), f"{p}.ctx.f", (rows, H), {"shape": (rows, H)})
        proj = b.linear(ctxf, f"{p}.wo", f"{p}.bo", H, H, f"{p}.o.out")
        x_attn = b.emit("add", (x, proj), f"{p}.resid1", (rows, H))
        c = b.norm(x_attn, f"{p}.ln2", f"{p}.ln2.out")
        f1 = b.linear(c, f"{p}.w_fc1", f"{p}.b_fc1", H, cfg.intermediate_size, f"{p}.fc1.out")
        g = b.emit("gelu_tanh", (f1,), f"{p}.act", (rows, cfg.intermediate_size))
        f2 = b.linear(g, f"{p}.w_fc2", f"{p}.b_fc2", cfg.intermediate_size, H, f"{p}.fc2.out")
        x = b.emit("add", (x_attn, f2), f"{p}.resid2", (rows, H))

    M = H * cfg.merge_unit
    mrows = rows // cfg.merge_unit
    mn = b.norm(x, "m_ln", "merger.ln.out")
    mc = b.emit("reshape", (mn,), "merger.concat", (mrows, M), {"shape": (mrows, M)})
    m1 = b.linear(mc, "w_m1", "b_m1", M, M, "merger.fc1.out")
    mg = b.emit("gelu_erf", (m1,), "merger.act", (mrows, M))
    out = b.linear(mg, "w_m2", "b_m2", M, cfg.out_hidden_size, "merger.out")
    return Graph(tensors=b.tensors, ops=tuple(b.ops), inputs=(image,), outputs=(out,))


# --- host-side tables (reference hexlib/models/loader.py) -----------------

def vision_position_ids(grid: int, merge: int) -> np.ndarray:
    """(row, col) id per token, in merge-block order (`loader.py:81-94`)."""
    blocks = grid // merge
    rows = np.repeat(np.arange(grid), grid).reshape(grid, grid)
    cols = np.tile(np.arange(grid), grid).reshape(grid, grid)

    def order(a):
        return a.reshape(blocks, merge, blocks, merge).transpose(0, 2, 1, 3).reshape(-1)

    return np.stack([order(rows), order(cols)], axis=-1)


def rope_tables(cfg: VitConfig) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin `[tokens, head_dim]` float32 (`loader.py:97-117`): inv_freq over
    head_dim/4 frequencies, row and column angles concatenated to head_dim/2,
    then the whole half duplicated. Replicated per image when batch > 1."""
    half = cfg.head_dim // 2
    inv_freq = 1.0 / cfg.rope_theta ** (np.arange(0, half, 2, dtype=np.float64) / half)
    pos = vision_position_ids(cfg.grid, cfg.spatial_merge_size).astype(np.float64)
    ang = (pos[:, :, None] * inv_freq[None, None, :]).reshape(pos.shape[0], -1)
    emb = np.concatenate([ang, ang], axis=-1)
    cos, sin = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    if cfg.batch > 1:
        cos, sin = np.tile(cos, (cfg.batch, 1)), np.tile(sin, (cfg.batch, 1))
    return cos, sin


def bilinear_corners(grid: int, side: int, merge: int) -> tuple[np.ndarray, np.ndarray]:
    """Four-corner indices and weights resampling a `side x side` learned grid
    onto a `grid x grid` patch grid, in merge-block token order
    (`loader.py:30-78`)."""
    pos = np.linspace(0, side - 1, grid)
    lo = pos.astype(np.int64)
    hi = np.minimum(lo + 1, side - 1)
    frac = pos - lo
    idx = [
        (lo[:, None] * side + lo[None, :]), (lo[:, None] * side + hi[None, :]),
        (hi[:, None] * side + lo[None, :]), (hi[:, None] * side + hi[None, :]),
    ]
    wts = [
        (1 - frac)[:, None] * (1 - frac)[None, :], (1 - frac)[:, None] * frac[None, :],
        frac[:, None] * (1 - frac)[None, :], frac[:, None] * frac[None, :],
    ]
    blocks = grid // merge
    tok = (np.arange(grid)[:, None] * grid + np.arange(grid)[None, :])
    order = tok.reshape(blocks, merge, blocks, merge).transpose(0, 2, 1, 3).reshape(-1)
    return (np.stack([i.reshape(-1)[order] for i in idx]),
            np.stack([w.reshape(-1)[order] for w in wts]))


def pos_embed_table(cfg: VitConfig, table: np.ndarray) -> np.ndarray:
    """Bilinear resample of the learned position grid (`loader.py:120-146`)."""
    side = int(round(table.shape[0] ** 0.5))
    if side * side != table.shape[0]:
        raise ValueError(f"pos_embed table has {table.shape[0]} rows, not a square")
    idx, wts = bilinear_corners(cfg.grid, side, cfg.spatial_merge_size)
    out = np.zeros((idx.shape[1], table.shape[1]), dtype=np.float64)
    for i in range(4):
        out += table[idx[i]].astype(np.float64) * wts[i][:, None]
    out = out.astype(np.float32)
    return np.tile(out, (cfg.batch, 1)) if cfg.batch > 1 else out


def feeds_from_params(graph: Graph, cfg: VitConfig, get: Callable[[str], np.ndarray]) -> dict[str, np.ndarray]:
    """HF parameter names -> graph consts (`loader.py:149-227`): Linear weights
    transposed to [in, out], the fused qkv split q/k/v along its output rows,
    Conv3d weight flattened in (C, T, ph, pw) order, tables folded."""
    H = cfg.hidden_size
    feeds: dict[str, np.ndarray] = {}
    conv = get("patch_embed.proj.weight")
    feeds["w_patch_embed"] = conv.reshape(conv.shape[0], -1).T
    feeds["b_patch_embed"] = get("patch_embed.proj.bias")
    feeds["pos_embed"] = pos_embed_table(cfg, get("pos_embed.weight"))
    feeds["rope_cos"], feeds["rope_sin"] = rope_tables(cfg)
    for layer in range(cfg.depth):
        src, dst = f"blocks.{layer}", f"blk{layer}"
        qkv_w, qkv_b = get(f"{src}.attn.qkv.weight"), get(f"{src}.attn.qkv.bias")
        for i, which in enumerate("qkv"):
            feeds[f"{dst}.w{which}"] = qkv_w[i * H:(i + 1) * H].T
            feeds[f"{dst}.b{which}"] = qkv_b[i * H:(i + 1) * H]
        feeds[f"{dst}.wo"] = get(f"{src}.attn.proj.weight").T
        feeds[f"{dst}.bo"] = get(f"{src}.attn.proj.bias")
        feeds[f"{dst}.w_fc1"] = get(f"{src}.mlp.linear_fc1.weight").T
        feeds[f"{dst}.b_fc1"] = get(f"{src}.mlp.linear_fc1.bias")
        feeds[f"{dst}.w_fc2"] = get(f"{src}.mlp.linear_fc2.weight").T
        feeds[f"{dst}.b_fc2"] = get(f"{src}.mlp.linear_fc2.bias")
        for ln in ("1", "2"):
            feeds[f"{dst}.ln{ln}_w"] = get(f"{src}.norm{ln}.weight")
            feeds[f"{dst}.ln{ln}_b"] = get(f"{src}.norm{ln}.bias")
    feeds["m_ln_w"] = get("merger.norm.weight")
    feeds["m_ln_b"] = get("merger.norm.bias")
    feeds["w_m1"] = get("merger.linear_fc1.weight").T
    feeds["w_m2"] = get("merger.linear_fc2.weight").T
    feeds["b_m1"] = get("merger.linear_fc1.bias")
    feeds["b_m2"] = get("merger.linear_fc2.bias")
    _check_feeds(graph, feeds)
    return feeds


def _check_feeds(graph: Graph, feeds: dict[str, Any]) -> None:
    consts = {t.name for t in graph.tensors.values() if t.const}
    missing, extra = consts - set(feeds), set(feeds) - consts - set(graph.inputs)
    if missing or extra:
        raise ValueError(f"feeds missing {sorted(missing)[:6]} extra {sorted(extra)[:6]}")
    for name, value in feeds.items():
        want = graph.tensor(name).shape
        if tuple(np.shape(value)) != want:
            raise ValueError(f"feed {name!r} is {np.shape(value)}, graph declares {want}")


def fuse_qkv_feeds(feeds: Mapping[str, np.ndarray], cfg: VitConfig) -> dict[str, np.ndarray]:
    """Feeds of the reference graph (separate q/k/v linears) rewritten for
    attention="fused_qkv_rope": per block, w{q,k,v} [H, H] side by side as
    wqkv [H, 3H] and b{q,k,v} as bqkv [3H] -- the same values, so both graphs
    compute the same function."""
    out = dict(feeds)
    for layer in range(cfg.depth):
        p = f"blk{layer}"
        out[f"{p}.wqkv"] = np.concatenate([out.pop(f"{p}.w{w}") for w in "qkv"], axis=1)
        out[f"{p}.bqkv"] = np.concatenate([out.pop(f"{p}.b{w}") for w in "qkv"])
    return out


def synthetic_feeds(graph: Graph, cfg: VitConfig, seed: int = 0) -> dict[str, np.ndarray]:
    """Seeded synthetic inputs: image U[0,1] fp32; matmul weights N(0,0.02)
    generated AS fp16 values (held as float32 so any consumer sees the exact
    fp16 value); biases, norm bias and pos_embed N(0,0.02) fp32; norm weight
    1 + N(0,0.02); RoPE tables from the grid. Weights declared q4_0 are fed as
    the same dense fp16-valued array; the arena builder quantizes them."""
    rng = np.random.default_rng(seed)
    feeds: dict[str, np.ndarray] = {}
    for name in graph.inputs:
        t = graph.tensor(name)
        feeds[name] = rng.random(t.shape, dtype=np.float32)
    cos, sin = rope_tables(cfg)
    for t in sorted((t for t in graph.tensors.values() if t.const), key=lambda t: t.name):
        if t.name == "rope_cos":
            feeds[t.name] = cos
        elif t.name == "rope_sin":
            feeds[t.name] = sin
        elif t.name == "pos_embed":
            base = (rng.standard_normal((cfg.num_tokens, t.shape[1])) * 0.02).astype(np.float32)
            feeds[t.name] = np.tile(base, (cfg.batch, 1)) if cfg.batch > 1 else base
        elif t.name.endswith("_w") and len(t.shape) == 1:
            w = 1.0 + rng.standard_normal(t.shape) * 0.02
            feeds[t.name] = w.astype(np.float16 if t.dtype == "fp16" else np.float32).astype(np.float32)
        elif len(t.shape) == 1:
            feeds[t.name] = (rng.standard_normal(t.shape) * 0.02).astype(np.float32)
        else:
            feeds[t.name] = (rng.standard_normal(t.shape) * 0.02).astype(np.float16).astype(np.float32)
    _check_feeds(graph, feeds)
    return feeds
