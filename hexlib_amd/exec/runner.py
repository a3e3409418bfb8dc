"""Kernel variants, their wire ids, and host-side variant selection.

Restates the reference's `RunnerSpec` table and `select`
(`hexlib/exec/runner.py:149-687`) and `KIND_ID` (`hexlib/runtime/genentry.py:67-88`):
one declarative record per kernel VARIANT giving its input dtypes, output dtype,
the scalars its C signature takes (derived on the device side from tensor
extents, or carried as op params for attrs), attr requirements, and per-buffer
layouts. The C entry adapters are generated from this table
(`hexlib_amd.exec.genentry`), so the two cannot disagree about argument order.

Ids 1-12 are the reference's and never move. Appended for this build:
13 rmsnorm, 14 matmul_epilogue_f16w (fp16 weight), 15 matmul_epilogue_q4k
(q4_0 grouped along K of W^T), 16 transpose_bth (perm (0,2,1,3), the batched
form of transpose_th), 17 matmul_epilogue_f16wt (fp16 weight stored W^T).

Each spec also names `extents`: the minimum element count of every buffer as a
C expression in the scalar names. The generated entry refuses a batch whose
tensors are smaller than the kernel will touch -- the DSP path never checked
this, but a GPU kernel reading past a buffer can fault the device.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping, Sequence

from hexlib_amd.exec.wire import LAYOUT_ID, float_param

WIRE_DENSE = ("fp32", "fp16", "int32")
WIRE_RAW = ("q4_0", "q8_0")

KIND_ID: dict[str, int] = {
    "add": 1,
    "cast": 2,
    "layernorm": 3,
    "matmul": 4,
    "matmul_epilogue": 5,
    "patchify": 6,
    "reshape": 7,
    "rope_2d": 8,
    "scale": 9,
    "softmax": 10,
    "transpose": 11,
    "transpose_hd": 12,
    "rmsnorm": 13,
    "matmul_epilogue_f16w": 14,
    "matmul_epilogue_q4k": 15,
    "transpose_bth": 16,
    "matmul_epilogue_f16wt": 17,
    "attention": 18,
    "attention_qk_v": 19,
    "rope_2d_qk": 20,
    "matmul_epilogue_f16wt_res": 21,
    "matmul_epilogue_f16wt_rope": 22,
    "attention_qkv": 23,
    "layernorm_matmul_epilogue_f16wt": 24,
    "matmul_epilogue_q8k": 25,
    "lnfold_matmul_epilogue_f16wt": 26,
    "lnfold_matmul_epilogue_f16wt_rope": 27,
    "matmul_epilogue_res": 28,
    "matmul_epilogue_q8k_res": 29,
    "matmul_epilogue_q4k_res": 30,
    "matmul_epilogue_q8k_rope": 31,
}


@dataclass(frozen=True)
class Scalar:
    """One argument of the C signature after the buffers.

    `source`: 'attr:<name>' (op param), 'numel:<i>', 'dim:<i>:<axis>' or
    'rows:<i>:<axis>' (derived from buffer i's extents on the device side,
    reference `runner.py:149-226`). `name` is the C identifier the generated
    entry binds it to. `codes` maps a string attr to an int code; `default`
    is used when a zero-filled param slot arrives (only for int attrs that
    extend a reference signature, e.g. patchify's batch)."""

    source: str
    ctype: str = "int"
    name: str = ""
    codes: tuple[tuple[str, int], ...] = ()
    default: int | None = None

    def value(self, shapes: Sequence[tuple[int, ...]], attrs: Mapping[str, Any]):
        kind, _, rest = self.source.partition(":")
        if kind == "attr":
            if rest not in attrs:
                if self.default is not None:
                    return self.default
                raise KeyError(f"scalar wants attr {rest!r}; op attrs are {sorted(attrs)}")
            v = attrs[rest]
            if self.codes:
                table = dict(self.codes)
                if v not in table:
                    raise ValueError(f"{self.source}: {v!r} is not one of {sorted(table)}")
                return table[v]
            return v
        if kind == "numel":
            n = 1
            for d in shapes[int(rest)]:
                n *= int(d)
            return n
        idx, _, axis = rest.partition(":")
        shape = tuple(shapes[int(idx)]) + (1,) * 4
        if kind == "dim":
            return int(shape[int(axis)])
        if kind == "rows":
            ext = int(shape[int(axis)])
            total = 1
            for d in shapes[int(idx)]:
                total *= int(d)
            if ext <= 0:
                raise ValueError(f"{self.source}: zero extent")
            return total // ext
        raise ValueError(f"unknown scalar source {self.source!r}")


@dataclass(frozen=True)
class RunnerSpec:
    kind: str
    entry: str                      # C function the entry calls (kernel_api.h name)
    inputs: tuple[str, ...]
    out_dtype: str
    scalars: tuple[Scalar, ...] = ()
    requires: tuple[tuple[str, Any], ...] = ()
    layouts: tuple[str, ...] = ()
    extents: tuple[str, ...] = ()   # min element count per buffer (C expressions)
    checks: tuple[str, ...] = ()    # C conditions on the scalars / buffers, else ERR_INVAL_PARAMS
    rank: int | None = None         # rank of input 0 the scalar sources assume (None: any)
    weight: tuple[int, str] | None = None   # (input index, dtype) this variant is chosen by
    primary: bool = True            # the reference's own variant when several match
    notes: str = ""

    def __post_init__(self) -> None:
        for dt in self.inputs:
            if dt not in WIRE_DENSE and dt not in WIRE_RAW:
                raise ValueError(f"{self.kind}: unknown input dtype {dt!r}")
        if self.out_dtype not in WIRE_DENSE:
            raise ValueError(f"{self.kind}: output must be dense, got {self.out_dtype!r}")
        if self.layouts:
            if len(self.layouts) != len(self.inputs) + 1:
                raise ValueError(f"{self.kind}: need one layout per buffer")
            for lay in self.layouts:
                if lay not in LAYOUT_ID:
                    raise ValueError(f"{self.kind}: unknown layout {lay!r}")
        if self.extents and len(self.extents) != len(self.inputs) + 1:
            raise ValueError(f"{self.kind}: need one extent per buffer")

    def buf_layouts(self) -> tuple[str, ...]:
        return self.layouts or ("row_major",) * (len(self.inputs) + 1)

    def accepts(self, attrs: Mapping[str, Any]) -> bool:
        return all(attrs.get(k) == v for k, v in self.requires)

    def check_rank(self, shapes: Sequence[tuple[int, ...]]) -> None:
        """The wire pads `ne` to four with ones, so a spec's `dim:`/`rows:`
        sources silently mean different axes at another rank; refuse it on the
        host rather than run a correctly-shaped wrong answer."""
        if self.rank is not None and len(shapes[0]) != self.rank:
            raise ValueError(f"{self.entry} takes a rank-{self.rank} input 0, got shape {tuple(shapes[0])}")

    def check_requires(self, attrs: Mapping[str, Any]) -> None:
        for key, want in self.requires:
            if attrs.get(key) != want:
                raise ValueError(f"{self.entry} implements {self.kind} only for {key}={want!r}, "
                                 f"this op has {key}={attrs.get(key)!r}")

    def params(self, shapes: Sequence[tuple[int, ...]], attrs: Mapping[str, Any]) -> tuple[int, ...]:
        """The op-param words: attr-sourced scalars only, floats as IEEE bits
        (reference `hexlib/exec/dsp.py:286-305`)."""
        out: list[int] = []
        for sc in self.scalars:
            if not sc.source.startswith("attr:"):
                continue
            v = sc.value(shapes, attrs)
            out.append(int(v) if sc.ctype == "int" else float_param(v))
        return tuple(out)


def _S(source, name, ctype="int", **kw):
    return Scalar(source=source, ctype=ctype, name=name, **kw)


_ACT_CODES = (("none", 0), ("gelu_tanh", 1), ("gelu_erf", 2))
_MM_SCALARS = (_S("dim:0:0", "M"), _S("dim:0:1", "K"), _S("dim:1:1", "N"),
               _S("attr:act", "act", codes=_ACT_CODES))

SPECS: dict[str, RunnerSpec] = {
    "scale": RunnerSpec(
        "scale", "scale_fp16", ("fp16",), "fp16",
        (_S("numel:0", "n"), _S("attr:factor", "factor", "float")),
        extents=("n", "n")),
    "add": RunnerSpec(
        "add", "add_fp16", ("fp16", "fp16"), "fp16", (_S("numel:0", "n"),),
        extents=("n", "n", "n"),
        notes="the pos_embed add takes an fp32 operand rounded to fp16 at staging"),
    "cast": RunnerSpec(
        "cast", "cast_f32_f16", ("fp32",), "fp16", (_S("numel:0", "n"),),
        requires=(("dtype", "fp16"),), extents=("n", "n")),
    "transpose": RunnerSpec(
        "transpose", "transpose_th_fp16", ("fp16",), "fp16",
        (_S("dim:0:0", "T"), _S("dim:0:1", "H"), _S("dim:0:2", "D")),
        requires=(("perm", (1, 0, 2)),), extents=("(uint64_t)T*H*D", "(uint64_t)T*H*D"),
        rank=3),
    "transpose_hd": RunnerSpec(
        "transpose", "transpose_hd_fp16", ("fp16",), "fp16",
        (_S("dim:0:0", "B"), _S("dim:0:1", "T"), _S("dim:0:2", "D")),
        requires=(("perm", (0, 2, 1)),), extents=("(uint64_t)B*T*D", "(uint64_t)B*T*D"),
        rank=3),
    "transpose_bth": RunnerSpec(
        "transpose", "transpose_bth_fp16", ("fp16",), "fp16",
        (_S("dim:0:0", "B"), _S("dim:0:1", "T"), _S("dim:0:2", "H"), _S("dim:0:3", "D")),
        requires=(("perm", (0, 2, 1, 3)),),
        extents=("(uint64_t)B*T*H*D", "(uint64_t)B*T*H*D"),
        notes="extension: [B,T,H,D] -> [B,H,T,D], the batched transpose_th",
        rank=4),
    "patchify": RunnerSpec(
        "patchify", "patchify_fp32_batched", ("fp32",), "fp32",
        (_S("dim:0:0", "BC"), _S("dim:0:1", "T"), _S("dim:0:2", "H"), _S("dim:0:3", "W"),
         _S("attr:patch", "patch"), _S("attr:merge", "merge"),
         _S("attr:grid_h", "grid_h"), _S("attr:grid_w", "grid_w"),
         _S("attr:batch", "batch", default=1)),
        extents=("(uint64_t)BC*T*H*W",
                 "(uint64_t)(batch > 0 ? batch : 1)*grid_h*grid_w*(BC/(batch > 0 ? batch : 1))*T*patch*patch"),
        notes="params[4] = batch (0 or 1 = one image, reference blobs zero-fill it); "
              "the image is [batch*C, T, H, W]",
        rank=4),
    "matmul": RunnerSpec(
        "matmul", "matmul_fp16", ("fp16", "fp16"), "fp16",
        (_S("dim:0:0", "Bn"), _S("dim:0:1", "M"), _S("dim:0:2", "K"), _S("dim:1:2", "N")),
        extents=("(uint64_t)Bn*M*K", "(uint64_t)Bn*K*N", "(uint64_t)Bn*M*N"),
        rank=3),
    "matmul_epilogue": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_fp16", ("fp16", "q4_0", "fp32"), "fp16",
        _MM_SCALARS, extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        weight=(1, "q4_0"),
        notes="q4_0 weight [K, N], blocks along N (the reference kernel ABI)",
        rank=2),
    "matmul_epilogue_q4k": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_q4k_fp16", ("fp16", "q4_0", "fp32"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "q4_0_kgroup", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        weight=(1, "q4_0"), primary=False,
        notes="q4_0 weight, logical [K, N] on the wire, stored as W^T [N, K] blocked along K",
        rank=2),
    "matmul_epilogue_q8k": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_q8k_fp16", ("fp16", "q8_0", "fp32"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "q8_0_kgroup", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        checks=("K % 32 == 0", "((uintptr_t)a->buf[1] & 1) == 0"),
        weight=(1, "q8_0"), primary=False,
        notes="extension: q8_0 weight, logical [K, N] on the wire, stored as W^T [N, K] blocked along K "
              "(the reference has the dtype, no kernel)"),
    "matmul_epilogue_res": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_res_fp16", ("fp16", "q4_0", "fp32", "fp16"), "fp16",
        _MM_SCALARS, extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N", "(uint64_t)M*N"),
        weight=(1, "q4_0"), primary=False,
        notes="extension: the reference-ABI q4_0 linear (blocks along N) with the residual add that "
              "consumes it folded into the epilogue (fuse_residual)",
        rank=2),
    "matmul_epilogue_q8k_res": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_q8k_res_fp16", ("fp16", "q8_0", "fp32", "fp16"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "q8_0_kgroup", "row_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N", "(uint64_t)M*N"),
        checks=("K % 32 == 0", "((uintptr_t)a->buf[1] & 1) == 0"),
        weight=(1, "q8_0"), primary=False,
        notes="extension: the q8_0 (K-grouped W^T) linear with the residual add in the epilogue",
        rank=2),
    "matmul_epilogue_q4k_res": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_q4k_res_fp16", ("fp16", "q4_0", "fp32", "fp16"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "q4_0_kgroup", "row_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N", "(uint64_t)M*N"),
        weight=(1, "q4_0"), primary=False,
        notes="extension: the K-grouped q4_0 linear with the residual add in the epilogue",
        rank=2),
    "matmul_epilogue_f16w": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_f16w_fp16", ("fp16", "fp16", "fp32"), "fp16",
        _MM_SCALARS, extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        weight=(1, "fp16"), primary=False,
        notes="fp16 weight [K, N] row-major",
        rank=2),
    "matmul_epilogue_f16wt": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_f16wt_fp16", ("fp16", "fp16", "fp32"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "col_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        weight=(1, "fp16"), primary=False,
        notes="fp16 weight, logical [K, N] on the wire, stored as W^T [N, K] (K contiguous)",
        rank=2),
    "softmax": RunnerSpec(
        "softmax", "softmax_fp16", ("fp16",), "fp16",
        (_S("rows:0:2", "R"), _S("dim:0:2", "C")), requires=(("axis", -1),),
        extents=("(uint64_t)R*C", "(uint64_t)R*C"),
        rank=3),
    "rope_2d": RunnerSpec(
        "rope_2d", "rope_2d_fp16", ("fp16", "fp32", "fp32"), "fp16",
        (_S("dim:0:0", "T"), _S("dim:0:1", "H"), _S("dim:0:2", "D")),
        extents=("(uint64_t)T*H*D", "(uint64_t)T*D", "(uint64_t)T*D", "(uint64_t)T*H*D"),
        rank=3),
    "layernorm": RunnerSpec(
        "layernorm", "layernorm_fp16", ("fp16", "fp32", "fp32"), "fp16",
        (_S("rows:0:1", "R"), _S("dim:0:1", "C"), _S("attr:eps", "eps", "float")),
        extents=("(uint64_t)R*C", "C", "C", "(uint64_t)R*C"),
        rank=2),
    "rmsnorm": RunnerSpec(
        "rmsnorm", "rmsnorm_fp16", ("fp16", "fp16"), "fp16",
        (_S("rows:0:1", "R"), _S("dim:0:1", "C"), _S("attr:eps", "eps", "float")),
        extents=("(uint64_t)R*C", "C", "(uint64_t)R*C"),
        rank=2),
    "attention": RunnerSpec(
        "attention", "attention_fp16", ("fp16", "fp16", "fp16"), "fp16",
        (_S("dim:0:0", "rows"), _S("dim:0:1", "H"), _S("dim:0:2", "D"),
         _S("attr:batch", "batch"), _S("attr:scale", "scale", "float")),
        extents=("(uint64_t)rows*H*D",) * 4,
        checks=("D == 32 || D == 64", "rows % batch == 0", "(uint64_t)batch * H <= 65535",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0",
                "((uintptr_t)a->buf[2] & 15) == 0", "((uintptr_t)a->buf[3] & 15) == 0"),
        rank=3,
        notes="extension: fused softmax(scale q k^T) v over [batch*T, H, D] q/k/v"),
    "matmul_epilogue_f16wt_res": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_f16wt_res_fp16", ("fp16", "fp16", "fp32", "fp16"), "fp16",
        _MM_SCALARS,
        layouts=("row_major", "col_major", "row_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*N", "(uint64_t)M*N"),
        weight=(1, "fp16"), primary=False, rank=2,
        notes="extension: a linear with the residual add that consumes it folded into the "
              "epilogue (fused by hexlib_amd.graph.fuse.fuse_residual); fp16 W^T only"),
    "matmul_epilogue_f16wt_rope": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_f16wt_rope_fp16", ("fp16", "fp16", "fp32", "fp32", "fp32"), "fp16",
        _MM_SCALARS + (_S("attr:rope_heads", "rope_heads"), _S("attr:rope_dim", "rope_dim")),
        layouts=("row_major", "col_major_rope", "row_major", "col_major", "col_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*rope_dim", "(uint64_t)M*rope_dim",
                 "(uint64_t)M*N"),
        checks=("K % 64 == 0", "N % 4 == 0", "rope_dim % 4 == 0", "2LL * rope_heads * rope_dim <= N",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0",
                "((uintptr_t)a->buf[5] & 7) == 0"),
        weight=(1, "fp16"), primary=False, rank=2,
        notes="extension: the fused q/k/v linear with rope_2d on its q and k heads in the epilogue "
              "(fused by hexlib_amd.graph.fuse.fuse_rope)"),
    "layernorm_matmul_epilogue_f16wt": RunnerSpec(
        "layernorm_matmul_epilogue", "layernorm_matmul_epilogue_f16wt_fp16",
        ("fp16", "fp32", "fp32", "fp16", "fp32"), "fp16",
        (_S("dim:0:0", "M"), _S("dim:0:1", "K"), _S("dim:3:1", "N"), _S("attr:act", "act", codes=_ACT_CODES),
         _S("attr:eps", "eps", "float")),
        layouts=("row_major", "row_major", "row_major", "col_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "K", "K", "(uint64_t)K*N", "N", "(uint64_t)M*N"),
        checks=("K >= 512", "K <= 768", "K % 64 == 0",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[3] & 15) == 0"),
        weight=(3, "fp16"), rank=2,
        notes="extension: layernorm over K then the W^T linear, one launch "
              "(fused by hexlib_amd.graph.fuse.fuse_layernorm)"),
    "matmul_epilogue_q8k_rope": RunnerSpec(
        "matmul_epilogue", "matmul_epilogue_q8k_rope_fp16", ("fp16", "q8_0", "fp32", "fp32", "fp32"), "fp16",
        _MM_SCALARS + (_S("attr:rope_heads", "rope_heads"), _S("attr:rope_dim", "rope_dim")),
        layouts=("row_major", "q8_0_kgroup_rope", "row_major", "col_major", "col_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "N", "(uint64_t)M*rope_dim", "(uint64_t)M*rope_dim",
                 "(uint64_t)M*N"),
        checks=("K % 256 == 0", "N % 4 == 0", "rope_dim % 4 == 0", "2LL * rope_heads * rope_dim <= N",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 1) == 0",
                "((uintptr_t)a->buf[5] & 7) == 0"),
        weight=(1, "q8_0"), primary=False, rank=2,
        notes="extension: the fused q/k/v linear with q8_0 weights and rope_2d on its q and k heads in "
              "the epilogue (fuse_rope)"),
    "lnfold_matmul_epilogue_f16wt": RunnerSpec(
        "lnfold_matmul_epilogue", "lnfold_matmul_epilogue_f16wt_fp16", ("fp16", "fp16", "fp32"), "fp16",
        _MM_SCALARS + (_S("attr:eps", "eps", "float"),),
        layouts=("row_major", "col_major", "row_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "2*(uint64_t)N", "(uint64_t)M*N"),
        checks=("K % 256 == 0",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0"),
        weight=(1, "fp16"), primary=False, rank=2,
        notes="extension: a layernorm folded into the W^T linear that consumes it "
              "(hexlib_amd.graph.fuse.fold_layernorm): weight-scaled W', bias2 = [c2 | c1]"),
    "lnfold_matmul_epilogue_f16wt_rope": RunnerSpec(
        "lnfold_matmul_epilogue", "lnfold_matmul_epilogue_f16wt_rope_fp16",
        ("fp16", "fp16", "fp32", "fp32", "fp32"), "fp16",
        _MM_SCALARS + (_S("attr:rope_heads", "rope_heads"), _S("attr:rope_dim", "rope_dim"),
                       _S("attr:eps", "eps", "float")),
        layouts=("row_major", "col_major_rope", "row_major", "col_major", "col_major", "row_major"),
        extents=("(uint64_t)M*K", "(uint64_t)K*N", "2*(uint64_t)N", "(uint64_t)M*rope_dim",
                 "(uint64_t)M*rope_dim", "(uint64_t)M*N"),
        checks=("K % 256 == 0", "N % 4 == 0", "rope_dim % 4 == 0",
                "2LL * rope_heads * rope_dim <= N",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0",
                "((uintptr_t)a->buf[5] & 7) == 0"),
        weight=(1, "fp16"), primary=False, rank=2,
        notes="extension: the folded layernorm with the q/k rope of the fused q/k/v linear in the "
              "epilogue (fold_layernorm after fuse_rope)"),
    "attention_qkv": RunnerSpec(
        "attention", "attention_qkv_fp16", ("fp16",), "fp16",
        (_S("dim:0:0", "rows"), _S("dim:0:2", "H"), _S("dim:0:3", "D"),
         _S("attr:batch", "batch"), _S("attr:scale", "scale", "float")),
        extents=("(uint64_t)rows*3*H*D", "(uint64_t)rows*H*D"),
        checks=("a->ne[0][1] == 3", "D == 32 || D == 64", "rows % batch == 0",
                "(uint64_t)batch * H <= 65535",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0"),
        rank=4,
        notes="extension: attention with q, k, v from one [rows, 3, H, D] tensor"),
    "attention_qk_v": RunnerSpec(
        "attention", "attention_qk_v_fp16", ("fp16", "fp16"), "fp16",
        (_S("dim:0:0", "rows"), _S("dim:0:2", "H"), _S("dim:0:3", "D"),
         _S("attr:batch", "batch"), _S("attr:scale", "scale", "float")),
        extents=("(uint64_t)rows*2*H*D", "(uint64_t)rows*3*H*D", "(uint64_t)rows*H*D"),
        checks=("a->ne[0][1] == 2", "a->ne[1][0] == a->ne[0][0]", "a->ne[1][1] == 3",
                "a->ne[1][2] == a->ne[0][2]", "a->ne[1][3] == a->ne[0][3]",
                "D == 32 || D == 64", "rows % batch == 0", "(uint64_t)batch * H <= 65535",
                "((uintptr_t)a->buf[0] & 15) == 0", "((uintptr_t)a->buf[1] & 15) == 0",
                "((uintptr_t)a->buf[2] & 15) == 0"),
        rank=4,
        notes="extension: attention with q, k from rope_2d_qk's [rows, 2, H, D] and v from the "
              "fused [rows, 3, H, D] projection"),
    "rope_2d_qk": RunnerSpec(
        "rope_2d_qk", "rope_2d_qk_fp16", ("fp16", "fp32", "fp32"), "fp16",
        (_S("dim:0:0", "rows"), _S("dim:0:2", "H"), _S("dim:0:3", "D")),
        extents=("(uint64_t)rows*3*H*D", "(uint64_t)rows*D", "(uint64_t)rows*D", "(uint64_t)rows*2*H*D"),
        checks=("a->ne[0][1] == 3", "D % 2 == 0"),
        rank=4,
        notes="extension: rope_2d on the q and k parts of a fused [rows, 3, H, D] projection"),
}


class SelectError(ValueError):
    pass


def variants_for(kind: str) -> tuple[str, ...]:
    return tuple(n for n, s in SPECS.items() if s.kind == kind)


def select(kind: str, attrs: Mapping[str, Any], in_dtypes: Sequence[str] | None = None,
           weight_layout: str | None = None) -> tuple[str, RunnerSpec]:
    """The variant serving this op, as `(name, spec)` (reference `runner.py:641-687`).

    Attrs filter by `requires`. When the caller knows its input dtypes, variants
    keyed on a weight dtype are filtered by it (fp16 vs q4_0 weights), and a
    `weight_layout` picks between layouts of the same dtype. Ambiguity left
    after that resolves to the reference's own (`primary`) variant, or is an
    error -- never a dict-order coin flip."""
    cands = [(n, s) for n, s in SPECS.items() if s.kind == kind]
    if not cands:
        raise SelectError(f"no kernel implements {kind!r}")
    ok = [(n, s) for n, s in cands if s.accepts(attrs)]
    if in_dtypes is not None:
        ok = [(n, s) for n, s in ok
              if len(s.inputs) == len(in_dtypes)
              and (s.weight is None or in_dtypes[s.weight[0]] == s.weight[1])]
    if weight_layout is not None and len(ok) > 1:
        narrowed = [(n, s) for n, s in ok
                    if s.weight is None or s.buf_layouts()[s.weight[0]] == weight_layout]
        ok = narrowed or ok
    if len(ok) > 1:
        primary = [(n, s) for n, s in ok if s.primary]
        if len(primary) == 1:
            ok = primary
    if len(ok) > 1:
        # same weight dtype, several storage layouts: the plain row-major ABI
        plain = [(n, s) for n, s in ok
                 if s.weight is not None and s.buf_layouts()[s.weight[0]] == "row_major"]
        if len(plain) == 1:
            ok = plain
    if len(ok) == 1:
        return ok[0]
    if not ok:
        raise SelectError(f"no {kind!r} kernel accepts attrs {dict(attrs)} / dtypes {in_dtypes}; "
                          f"candidates {[n for n, _ in cands]}")
    raise SelectError(f"{kind!r} is ambiguous between {[n for n, _ in ok]}")
