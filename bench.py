"""Benchmark: encoder images/sec @256x256 fp16 on one MI355X, with per-op
roofline fractions and the CPU oracle timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-suite]

A step is one whole-plan replay of the ViT encoder (BASELINE cfg 4: 12
blocks, hidden 768, 12 heads, MLP 3072, LayerNorm, 2D RoPE, merger) over one
256x256 image, replayed as ONE captured hipGraph through the session's batch
invoke. The plan is the product default: per block, one [768, 2304] q/k/v
linear, one rope op for q and k and one fused attention op (127 launches); the
reference graph's unfused plan (259 launches) is reported as a variant.
Inputs and weights are resident in HBM
before timing starts. `value` is images/sec over exactly K replays bracketed
by device synchronisation.

Per-op durations come from the same product path: a blob that repeats one op
R times, captured as a hipGraph and timed with HIP events on the session
stream (cycles_total of a TIMED invoke), divided by R. "in_plan" figures use
the plan's own buffers (cache-warm, as in the encoder); the "suite" figures
rotate R distinct buffer sets whose footprint exceeds 512 MB (above the
256 MB MALL), so they measure HBM, at BASELINE cfg 2/3 shapes.

Roofline peaks: HBM 8 TB/s; dense fp16 MFMA 2.5 PFLOP/s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import replace

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
METRIC = "encoder images/sec @256x256 fp16, 1 GPU; per-op % of MFMA/HBM roofline"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---- algorithmic work per op --------------------------------------------------------

_ESZ = {"fp16": 2, "fp32": 4}
_ATTN_BATCH: dict = {}   # attention input shape -> images per call, filled from the plan


def op_work(spec_name: str, in_shapes, out_shape, in_dtypes, out_dtype) -> tuple[str, float]:
    """('mfma', flops) for GEMMs, ('hbm', bytes) for everything else: every
    input read once and every output written once."""
    def nb(shape, dt):
        n = int(np.prod(shape))
        return n // 32 * 18 if dt == "q4_0" else n * _ESZ[dt]
    if spec_name == "matmul":
        bn, m, k = in_shapes[0]
        n = in_shapes[1][-1]
        return "mfma", 2.0 * bn * m * k * n
    if spec_name.startswith("attention"):   # q.k^T and p.v per (image, head); batch from the plan
        rows, h, d = in_shapes[0][0], in_shapes[0][-2], in_shapes[0][-1]
        t = rows // max(1, _ATTN_BATCH.get(tuple(in_shapes[0]), 1))
        return "mfma", 4.0 * rows * t * h * d
    if spec_name.startswith(("matmul_epilogue", "lnfold_matmul_epilogue")):   # (x, W, bias ...)
        m, k = in_shapes[0]
        n = in_shapes[1][-1]
        return "mfma", 2.0 * m * k * n
    if spec_name.startswith("layernorm_matmul_epilogue"):   # (x, ln_w, ln_b, w, bias)
        m, k = in_shapes[0]
        n = in_shapes[3][-1]
        return "mfma", 2.0 * m * k * n
    total = sum(nb(s, d) for s, d in zip(in_shapes, in_dtypes)) + nb(out_shape, out_dtype)
    return "hbm", float(total)


def gemm_bytes(in_shapes, in_dtypes, out_shape) -> float:
    def nb(shape, dt):
        n = int(np.prod(shape))
        return n // 32 * 18 if dt == "q4_0" else n * _ESZ[dt]
    return sum(nb(s, d) for s, d in zip(in_shapes, in_dtypes)) + nb(out_shape, "fp16")


# ---- plan helpers -------------------------------------------------------------------------

def fold_rule(rows: int) -> bool:
    """Where folding a LayerNorm into its linear pays on MI355X: at every row
    count the encoder has. The folded op takes the K-across-waves form where
    its 64x64 tiles fit a round of CUs (batch 1 at 256x256), the tiled 64x64
    form above that (448x448: 784 rows) and the large-tile form where its
    128-row tiles fill a round (batch 32), as the unfused linear would; each
    measured faster folded than unfolded (A/B on one box)."""
    return rows > 0


FOLD_LN_ROWS = fold_rule


def build_plan(cfg, seed=0, weight_layout="auto", residual=True, rope=True, layernorm=False,
               fold_ln_rows=None):
    """The product plan: fusions on (`residual` folds residual adds into the
    fp16 linears, `rope` the q/k rope into the fused q/k/v linear; the
    config's `attention` picks the attention form). Each LayerNorm whose row
    count `fold_ln_rows` admits (default FOLD_LN_ROWS: `fold_rule`) is folded
    algebraically into the linear it feeds (`fold_layernorm`: no launch of its
    own). `layernorm` (the normalised rows recomputed in the
    linear's prologue) is off: every workgroup of that
    kernel normalises its whole row block again, 48 times per row at fc1,
    which costs more than the separate launch it saves (18.6 us against
    9.4 + 2.5 us on MI355X; a K-across-waves form with the row block resident
    measured 15.9 us, its LDS reads of the row spread over 8 KB slices
    conflicting 8 ways)."""
    from hexlib_amd import encoder as E
    from hexlib_amd.exec.wholeplan import build_whole_plan_batch
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=seed)
    fold = FOLD_LN_ROWS if fold_ln_rows is None else fold_ln_rows
    return g, feeds, build_whole_plan_batch(g, feeds, weight_layout=weight_layout,
                                            residual=residual and cfg.attention != "unfused",
                                            rope=rope and cfg.attention == "fused_qkv_rope",
                                            layernorm=layernorm and cfg.attention != "unfused",
                                            fold_ln_rows=fold if cfg.attention != "unfused" else 0)


def time_replays(plan, steps: int, warmup: int) -> float:
    """Seconds for exactly `steps` graph replays, bracketed by device syncs."""
    import torch
    from hexlib_amd import lib as L
    flags = L.INVOKE_GRAPH | L.INVOKE_NOSYNC
    kinds = plan.kinds
    for _ in range(max(warmup, 1)):
        plan.session.invoke(plan.batch.blob, kinds, flags)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        plan.session.invoke(plan.batch.blob, kinds, flags)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def unique_ops(g, wb):
    """(spec, input shapes/dtypes, output) -> [count, first op desc index]."""
    out = {}
    for i, op in enumerate(wb.graph_ops):
        spec = wb.op_specs[i]
        ins = tuple((wb.placements[n].shape, wb.placements[n].dtype) for n in op.inputs)
        if spec.startswith("attention"):
            _ATTN_BATCH[tuple(ins[0][0])] = int(op.attrs.get("batch", 1))
        o = wb.placements[op.outputs[0]]
        key = (spec, ins, (o.shape, o.dtype))
        if key not in out:
            out[key] = [0, i, op]
        out[key][0] += 1
    return out


def repeat_op_blob(wb, op_index: int, reps: int) -> bytes:
    """The plan's blob with its op list replaced by `reps` copies of one op."""
    import struct
    from hexlib_amd.exec import wire
    blob = wb.blob
    hdr = list(struct.unpack_from(wire._HDR, blob))
    off_ops = hdr[8]
    op = blob[off_ops + op_index * wire.OP_SIZE: off_ops + (op_index + 1) * wire.OP_SIZE]
    body = bytearray(blob[:off_ops] + op * reps)
    struct.pack_into("<I", body, 8, len(body))
    struct.pack_into("<I", body, 20, reps)
    return bytes(body)


def time_blob(session, blob: bytes, n_ops: int, iters: int = 5) -> float:
    """Mean GPU ns of one replay of a captured blob (TIMED graph invoke)."""
    from hexlib_amd import lib as L
    from hexlib_amd.exec.gpu import blob_kinds
    kinds = blob_kinds(blob)
    session.invoke(blob, kinds, L.INVOKE_GRAPH)             # capture + first run
    ns = []
    for _ in range(iters):
        rsp = session.invoke(blob, kinds, L.INVOKE_GRAPH | L.INVOKE_TIMED)
        ns.append(rsp.cycles_total)
    return float(np.median(ns))


def per_op_in_plan(plan, g, reps: int = 40) -> list[dict]:
    rows = []
    for (spec, ins, (oshape, odt)), (count, idx, op) in unique_ops(g, plan.batch).items():
        blob = repeat_op_blob(plan.batch, idx, reps)
        ns = time_blob(plan.session, blob, reps) / reps
        bound, work = op_work(spec, [s for s, _ in ins], oshape, [d for _, d in ins], odt)
        rate = work / ns  # flops/ns = GFLOP/s ; bytes/ns = GB/s
        peak = MFMA_FP16_PEAK_TFLOPS * 1e3 if bound == "mfma" else HBM_PEAK_GBS
        rows.append({"op": spec, "shape": [list(s) for s, _ in ins], "count": count,
                     "avg_ns": round(ns, 1), "bound": bound,
                     "achieved": round(rate / 1e3, 3) if bound == "mfma" else round(rate, 1),
                     "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                     "frac": round(rate / peak, 4),
                     "total_us": round(count * ns / 1e3, 1)})
    return sorted(rows, key=lambda r: -r["total_us"])


# ---- roofline of the dominant kernel ---------------------------------------------------

def dominant_op(g, wb):
    """The plan's GEMM row with the most algorithmic work per image (launches
    x FLOPs; ties: first in plan order). For the cfg-4 encoder plan that is
    the MLP up-projection fc1, 256x768x3072 with its LayerNorm folded in (12
    launches, tied with fc2 in work and first in plan order)."""
    rows = []
    for (spec, ins, out), (count, idx, _) in unique_ops(g, wb).items():
        if not spec.startswith(("matmul_epilogue", "layernorm_matmul_epilogue", "lnfold_matmul_epilogue")):
            continue
        flops = op_work(spec, [s for s, _ in ins], out[0], [d for _, d in ins], out[1])[1]
        rows.append((count * flops, -idx, spec, ins, out, count))
    work, neg_idx, spec, ins, out, count = max(rows)
    return {"spec": spec, "index": -neg_idx, "count": count, "inputs": ins, "output": out}


def roofline(plan, g, reps: int = 200, iters: int = 7, cold: bool = True) -> dict:
    """Algorithmic work of one launch of the dominant op / its mean duration,
    measured with HIP events on the session stream around a captured graph of
    `reps` back-to-back launches (cycles_total of a TIMED invoke / reps).
    With `cold`, also the same linear over a >= 512 MiB operand rotation
    (`roofline_cold`); --roofline-only leaves it out, so that its rocprofv3
    trace holds the warm launches only."""
    d = dominant_op(g, plan.batch)
    shapes = [s for s, _ in d["inputs"]]
    dtypes = [t for _, t in d["inputs"]]
    oshape, odt = d["output"]
    flops = op_work(d["spec"], shapes, oshape, dtypes, odt)[1]
    nbytes = gemm_bytes(shapes, dtypes, oshape)
    blob = repeat_op_blob(plan.batch, d["index"], reps)
    ns = time_blob(plan.session, blob, reps, iters=iters) / reps
    ridge = MFMA_FP16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    ai = flops / nbytes
    m, k = shapes[0]
    n = oshape[-1]
    out = {"kernel": f"{d['spec']} {m}x{k}x{n}", "launches_per_image": d["count"],
           "avg_launch_ns": round(ns, 1), "algorithmic_bytes": int(nbytes), "flops": int(flops),
           "arith_intensity": round(ai, 1)}
    if ai < ridge:
        out.update({"bound": "hbm", "achieved": round(nbytes / ns, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(nbytes / ns / HBM_PEAK_GBS, 5)})
    else:
        out.update({"bound": "mfma", "achieved": round(flops / ns / 1e3, 3), "peak": MFMA_FP16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(flops / ns / 1e3 / MFMA_FP16_PEAK_TFLOPS, 5)})
    out["tflops"] = round(flops / ns / 1e3, 3)
    out["traffic"] = measured_traffic(out["kernel"])
    out["cache"] = (f"warm: {reps} back-to-back launches on the plan's own operands, which stay in "
                    f"L2 / the 256 MB last-level cache; 'cold' below rotates >= 512 MiB of distinct operands")
    if cold and d["spec"] in ("matmul_epilogue_f16wt", "lnfold_matmul_epilogue_f16wt"):
        out["cold"] = roofline_cold(plan.session, m, k, n, nbytes, flops, out["bound"],
                                    lnfold=d["spec"].startswith("lnfold"))
    return out


def roofline_cold(session, M: int, K: int, N: int, nbytes: int, flops: int, bound: str,
                  rotation_mib: int = 512, lnfold: bool = False) -> dict:
    """The dominant W^T linear (gelu epilogue, as fc1) over enough distinct
    (A, W^T, bias, out) sets that one pass touches >= rotation_mib MiB, more
    than the 256 MB last-level cache: each launch then reads its operands from
    HBM. The launches are captured into one graph on the session's stream and
    timed with HIP events around its replays; best of 5 replays / sets."""
    import ctypes
    import torch
    from hexlib_amd import lib as L
    lib = L.load()
    P = ctypes.c_void_p
    nb = 2 * N if lnfold else N   # the folded LayerNorm's bias2 = [c2 | c1]
    per_set = (M * K + N * K + M * N) * 2 + nb * 4
    nsets = -(-(rotation_mib << 20) // per_set)
    gen = torch.Generator(device="cuda").manual_seed(11)
    sets = [(torch.randn(M, K, device="cuda", generator=gen).half(),
             (torch.randn(N, K, device="cuda", generator=gen) * 0.02).half(),
             torch.randn(nb, device="cuda", generator=gen) * 0.02,
             torch.empty(M, N, device="cuda", dtype=torch.float16)) for _ in range(nsets)]

    def launch(a, w, b, o):
        if lnfold:
            lib.lnfold_matmul_epilogue_f16wt_fp16(P(a.data_ptr()), P(w.data_ptr()), P(b.data_ptr()),
                                                  P(o.data_ptr()), M, K, N, 1, ctypes.c_float(1e-6))
        else:
            lib.matmul_epilogue_f16wt_fp16(P(a.data_ptr()), P(w.data_ptr()), P(b.data_ptr()), P(o.data_ptr()),
                                           M, K, N, 1)
    stream = torch.cuda.Stream()
    saved = lib.hexlib_gpu_get_stream()
    try:
        with torch.cuda.stream(stream):
            lib.hexlib_gpu_set_stream(P(stream.cuda_stream))
            for a, w, b, o in sets[:2]:   # warm the code path outside the capture
                launch(a, w, b, o)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for a, w, b, o in sets:
                    launch(a, w, b, o)
            graph.replay()
            stream.synchronize()
            best = float("inf")
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                graph.replay()
                e1.record(stream)
                e1.synchronize()
                best = min(best, e0.elapsed_time(e1) * 1e6 / nsets)
            err = lib.hexlib_gpu_take_error()
            if err:
                raise RuntimeError(f"cold roofline launch failed: HIP error {err}")
    finally:
        lib.hexlib_gpu_set_stream(P(saved))
    del sets
    torch.cuda.empty_cache()
    out = {"sets": nsets, "rotation_bytes": nsets * per_set, "avg_launch_ns": round(best, 1)}
    if bound == "hbm":
        out.update({"achieved": round(nbytes / best, 1), "unit": "GB/s",
                    "frac": round(nbytes / best / HBM_PEAK_GBS, 5)})
    else:
        out.update({"achieved": round(flops / best / 1e3, 3), "unit": "TFLOP/s",
                    "frac": round(flops / best / 1e3 / MFMA_FP16_PEAK_TFLOPS, 5)})
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_dominant_gemm.json")


def measured_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of known size), when it
    was taken for this same kernel and shape; else None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("traffic_bytes") if t.get("kernel") == kernel else None


def copy_reference(mib: int = 512) -> None:
    """A plain device copy of known size (mib MiB read + mib MiB written),
    launched so that a --pmc run can scale FETCH_SIZE/WRITE_SIZE to bytes."""
    import torch
    src = torch.ones((mib << 20) // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)    # one elementwise kernel: reads and writes mib MiB
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def trace_summary(d: str) -> str:
    """Markdown summary of a rocprofv3 output directory: per-kernel duration
    statistics from *_kernel_stats.csv and, for --pmc runs, the mean counter
    value per dispatch of each kernel from *_counter_collection.csv."""
    import csv
    import glob
    lines = []
    for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)):
        lines += [f"### {os.path.relpath(path, d)}", "",
                  "| kernel | calls | avg ns | min ns | max ns | % |", "|---|---|---|---|---|---|"]
        for r in csv.DictReader(open(path)):
            lines.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']):.0f} | "
                         f"{r['MinNs']} | {r['MaxNs']} | {float(r['Percentage']):.2f} |")
        lines.append("")
    for path in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
        acc = {}
        for r in csv.DictReader(open(path)):
            key = (r["Kernel_Name"][:90], r["Counter_Name"], r.get("Grid_Size", ""))
            a = acc.setdefault(key, [0.0, 0])
            a[0] += float(r["Counter_Value"])
            a[1] += 1
        lines += [f"### {os.path.relpath(path, d)}", "",
                  "| kernel | grid | counter | dispatches | mean per dispatch |", "|---|---|---|---|---|"]
        for (k, c, grid), (tot, n) in sorted(acc.items()):
            lines.append(f"| `{k}` | {grid} | {c} | {n} | {tot / n:.1f} |")
        lines.append("")
    return "\n".join(lines)


# ---- cold-buffer per-op suite (BASELINE cfg 2 / cfg 3 shapes) -------------------------

def suite_cases():
    from hexlib_amd import encoder as E
    r = np.random.default_rng(0)
    cos, sin = E.rope_tables(E.QWEN35_VISION_FP16)
    h = lambda *s: (r.standard_normal(s)).astype(np.float16)
    return [
        ("rmsnorm", {"eps": 1e-6}, [h(256, 768), h(768)], (256, 768)),
        ("layernorm", {"eps": 1e-6}, [h(256, 768), np.ones(768, np.float32), np.zeros(768, np.float32)], (256, 768)),
        ("softmax", {"axis": -1}, [(h(12, 256, 256) * 0.125).astype(np.float16)], (12, 256, 256)),
        ("rope_2d", {}, [h(256, 12, 64), cos, sin], (256, 12, 64)),
        ("transpose", {"perm": (1, 0, 2)}, [h(256, 12, 64)], (12, 256, 64)),
        ("transpose", {"perm": (0, 2, 1)}, [h(12, 256, 64)], (12, 64, 256)),
        ("add", {}, [h(256, 768), h(256, 768)], (256, 768)),
        ("scale", {"factor": 0.125}, [h(256, 768)], (256, 768)),
        ("cast", {"dtype": "fp16"}, [r.standard_normal((256, 768)).astype(np.float32)], (256, 768)),
        ("patchify", {"patch": 16, "temporal_patch": 1, "merge": 2, "grid_h": 16, "grid_w": 16},
         [r.random((3, 1, 256, 256), dtype=np.float32)], (256, 768)),
        ("matmul_epilogue", {"act": "gelu_tanh"}, [h(256, 768), (h(768, 2304) * 0.02).astype(np.float16),
                                                   np.zeros(2304, np.float32)], (256, 2304)),
        ("matmul_epilogue", {"act": "none"}, [h(256, 768), (h(768, 768) * 0.02).astype(np.float16),
                                              np.zeros(768, np.float32)], (256, 768)),
        ("matmul_epilogue", {"act": "gelu_tanh"}, [h(256, 768), (h(768, 3072) * 0.02).astype(np.float16),
                                                   np.zeros(3072, np.float32)], (256, 3072)),
        ("matmul_epilogue", {"act": "none"}, [h(256, 3072), (h(3072, 768) * 0.02).astype(np.float16),
                                              np.zeros(768, np.float32)], (256, 768)),
        ("matmul", {}, [h(12, 256, 64), h(12, 64, 256)], (12, 256, 256)),
        ("matmul", {}, [h(12, 256, 256), h(12, 256, 64)], (12, 256, 64)),
    ]


def q4_gemm_sweep(reps: int = 20) -> list[dict]:
    """BASELINE cfg 5: the K-grouped q4_0 GEMM (`matmul_epilogue_q4k_fp16`,
    fp16 scales U(0.005, 0.02), uniform nibbles, A ~ N(0, 1), no bias) at
    M in {1, 16, 256} and K x N in {896 x 4864, 4864 x 896, 2048 x 2048}.
    Each figure is the mean launch time over a captured graph of `reps`
    launches on one set of buffers (cache-warm), best of 5 replays."""
    import ctypes
    import torch
    from hexlib_amd import lib as L
    lib = L.load()
    P = ctypes.c_void_p
    stream = lambda: lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
    r = np.random.default_rng(5)
    rows = []
    for M in (1, 16, 256):
        for Kd, N in ((896, 4864), (4864, 896), (2048, 2048)):
            nb = N * Kd // 32
            blocks = np.empty((nb, 18), np.uint8)
            blocks[:, :2] = r.uniform(0.005, 0.02, nb).astype(np.float16).view(np.uint8).reshape(-1, 2)
            blocks[:, 2:] = r.integers(0, 256, (nb, 16), dtype=np.uint8)
            wq = torch.from_numpy(blocks.reshape(-1)).cuda()
            a = torch.from_numpy(r.standard_normal((M, Kd)).astype(np.float16)).cuda()
            bias = torch.zeros(N, dtype=torch.float32, device="cuda")
            c = torch.empty(M, N, dtype=torch.float16, device="cuda")
            call = lambda: lib.matmul_epilogue_q4k_fp16(P(a.data_ptr()), P(wq.data_ptr()), P(bias.data_ptr()),
                                                        P(c.data_ptr()), M, Kd, N, 0)
            stream()
            call()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                stream()
                for _ in range(reps):
                    call()
            stream()
            g.replay()
            torch.cuda.synchronize()
            best = float("inf")
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                g.replay()
                e1.record()
                torch.cuda.synchronize()
                best = min(best, e0.elapsed_time(e1) * 1e6 / reps)
            del g
            if lib.hexlib_gpu_take_error() != 0:
                raise RuntimeError(f"q4 GEMM {M}x{Kd}x{N} reported an error")
            nbytes = nb * 18 + M * Kd * 2 + N * 4 + M * N * 2
            flops = 2.0 * M * Kd * N
            mfma = flops / nbytes > MFMA_FP16_PEAK_TFLOPS * 1e3 / HBM_PEAK_GBS
            rate = flops / best / 1e3 if mfma else nbytes / best
            peak = MFMA_FP16_PEAK_TFLOPS if mfma else HBM_PEAK_GBS
            row = {"shape": [M, Kd, N], "avg_ns": round(best, 1), "bound": "mfma" if mfma else "hbm",
                   "achieved": round(rate, 3 if mfma else 1), "unit": "TFLOP/s" if mfma else "GB/s",
                   "frac": round(rate / peak, 4), "algorithmic_bytes": nbytes}
            rows.append(row)
            log(f"cfg5 q4 {M}x{Kd}x{N}: {best:.0f} ns, {row['achieved']} {row['unit']} ({row['frac']*100:.1f}%)")
    torch.cuda.synchronize()
    lib.hexlib_gpu_set_stream(P(None))
    return rows


def q4n_gemm_rows(reps: int = 20) -> list[dict]:
    """The reference-ABI q4_0 GEMM (`matmul_epilogue_fp16`: q4_0 blocks of 32
    along N, `kernels/matmul_epilogue_fp16/kernel_api.h:68-109,188-190`) at
    the encoder's four linear shapes at batch 1 (M = 256), with the bias and
    activation of each linear. Weights from quantize_q4_0 of N(0, 0.02);
    activations N(0, 1). Mean launch time over a captured graph of `reps`
    launches on one buffer set (cache-warm), best of 5 replays; roofline by
    the shape's arithmetic intensity (q4_0 weight bytes K * N * 18 / 32)."""
    import ctypes
    import torch
    from hexlib_amd import lib as L
    from hexlib_amd.quant import pack_q4_0_nblocked
    lib = L.load()
    P = ctypes.c_void_p
    r = np.random.default_rng(7)
    rows = []
    for Kd, N, act in ((768, 2304, 0), (768, 768, 0), (768, 3072, 1), (3072, 768, 0)):
        M = 256
        w = pack_q4_0_nblocked((r.standard_normal((Kd, N)) * 0.02).astype(np.float32))
        wq = torch.frombuffer(bytearray(w), dtype=torch.uint8).cuda()
        a = torch.from_numpy(r.standard_normal((M, Kd)).astype(np.float16)).cuda()
        bias = torch.from_numpy((r.standard_normal(N) * 0.02).astype(np.float32)).cuda()
        c = torch.empty(M, N, dtype=torch.float16, device="cuda")
        call = lambda: lib.matmul_epilogue_fp16(P(a.data_ptr()), P(wq.data_ptr()), P(bias.data_ptr()),
                                                P(c.data_ptr()), M, Kd, N, act)
        lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
        call()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
            for _ in range(reps):
                call()
        lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
        g.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e6 / reps)
        del g
        if lib.hexlib_gpu_take_error() != 0:
            raise RuntimeError(f"q4_0 GEMM {M}x{Kd}x{N} reported an error")
        nbytes = len(w) + M * Kd * 2 + N * 4 + M * N * 2
        flops = 2.0 * M * Kd * N
        mfma = flops / nbytes > MFMA_FP16_PEAK_TFLOPS * 1e3 / HBM_PEAK_GBS
        rate = flops / best / 1e3 if mfma else nbytes / best
        peak = MFMA_FP16_PEAK_TFLOPS if mfma else HBM_PEAK_GBS
        row = {"op": "matmul_epilogue_fp16 (q4_0 along N)", "shape": [M, Kd, N], "act": act,
               "avg_ns": round(best, 1), "bound": "mfma" if mfma else "hbm",
               "achieved": round(rate, 3 if mfma else 1), "unit": "TFLOP/s" if mfma else "GB/s",
               "frac": round(rate / peak, 4), "tflops": round(flops / best / 1e3, 2),
               "algorithmic_bytes": nbytes}
        rows.append(row)
        log(f"q4_0 (N-blocked) {M}x{Kd}x{N}: {best:.0f} ns, {row['achieved']} {row['unit']} "
            f"({row['frac'] * 100:.1f}%)")
    lib.hexlib_gpu_set_stream(P(None))
    return rows


def suite(session, min_footprint=600 << 20, max_reps=4000) -> list[dict]:
    import torch
    from hexlib_amd.exec import wire
    from hexlib_amd.exec.runner import KIND_ID, select
    from hexlib_amd.exec.wholeplan import align_up
    rows = []
    fd = 11
    for kind, attrs, arrays, out_shape in suite_cases():
        dtypes = ["fp16" if a.dtype == np.float16 else "fp32" for a in arrays]
        name, spec = select(kind, attrs, dtypes)
        odt = spec.out_dtype
        blobs = [np.ascontiguousarray(a).tobytes() for a in arrays]
        onb = int(np.prod(out_shape)) * _ESZ[odt]
        sizes = [align_up(len(b)) for b in blobs] + [align_up(onb)]
        per = sum(sizes)
        reps = int(min(max_reps, max(8, -(-min_footprint // per))))
        reps = min(reps, (wire.MAX_TENSORS - 1) // (len(arrays) + 1))
        arena = torch.empty(per * reps, dtype=torch.uint8, device="cuda")
        one = bytearray(per)
        off = 0
        for b, s in zip(blobs, sizes):
            one[off:off + len(b)] = b
            off += s
        arena.view(reps, per).copy_(torch.frombuffer(one, dtype=torch.uint8).to("cuda").expand(reps, per))
        torch.cuda.synchronize()
        tensors, ops = [], []
        shapes = [a.shape for a in arrays]
        lays = spec.buf_layouts()
        for r in range(reps):
            base = r * per
            idx = []
            off = 0
            for i, (a, s) in enumerate(zip(arrays, sizes[:-1])):
                tensors.append(wire.TensorDesc(0, base + off, len(blobs[i]), dtypes[i], lays[i], wire.pad_ne(a.shape)))
                idx.append(len(tensors) - 1)
                off += s
            tensors.append(wire.TensorDesc(0, base + off, onb, odt, lays[-1], wire.pad_ne(out_shape)))
            ops.append(wire.OpDesc(KIND_ID[name], spec.params(shapes, attrs), tuple(idx), (len(tensors) - 1,)))
        blob = wire.pack_batch([wire.BufDesc(fd, per * reps)], tensors, ops)
        session.mmap(fd, arena.data_ptr(), per * reps)
        try:
            ns = time_blob(session, blob, reps) / reps
        finally:
            session.munmap(fd)
        bound, work = op_work(name, shapes, out_shape, dtypes, odt)
        rate = work / ns
        peak = MFMA_FP16_PEAK_TFLOPS * 1e3 if bound == "mfma" else HBM_PEAK_GBS
        row = {"op": name, "shape": [list(s) for s in shapes], "avg_ns": round(ns, 1), "bound": bound,
               "achieved": round(rate / 1e3, 3) if bound == "mfma" else round(rate, 1),
               "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "frac": round(rate / peak, 4),
               "footprint_mb": round(per * reps / 2**20), "reps": reps}
        if bound == "mfma":
            gb = gemm_bytes(shapes, dtypes, out_shape)
            attain = min(MFMA_FP16_PEAK_TFLOPS * 1e3, work / gb * HBM_PEAK_GBS)
            row["frac_of_attainable"] = round(rate / attain, 4)
        rows.append(row)
        log(f"suite {name} {shapes}: {ns:.0f} ns, {row['achieved']} {row['unit']} ({row['frac']*100:.1f}%)")
        del arena
        torch.cuda.empty_cache()
    return rows


# ---- batch-32 GEMMs against the vendor library ------------------------------------------

def library_matmul_ns(m: int, k: int, n: int, reps: int = 20) -> float:
    """Mean ns of torch.matmul (hipBLASLt) on the same fp16 shape, A [m,k] times
    a transposed [n,k] weight, fp32 accumulate, no epilogue: the attainable
    bar for the product GEMM. A captured graph of `reps` launches timed with
    events on torch's stream, best of 5 replays."""
    import torch
    a = torch.randn(m, k, dtype=torch.float16, device="cuda")
    w = torch.randn(n, k, dtype=torch.float16, device="cuda").mul_(0.02)
    out = torch.empty(m, n, dtype=torch.float16, device="cuda")
    torch.matmul(a, w.t(), out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            torch.matmul(a, w.t(), out=out)
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e6 / reps)
    del g
    return best


def plain_linear_ns(m: int, k: int, n: int, act: int = 0, reps: int = 20) -> float:
    """Mean ns of this library's matmul_epilogue_f16wt_fp16 (no residual, no
    rope) on one fp16 shape with torch-allocated operands: a captured graph of
    `reps` launches on torch's stream, best of 5 replays."""
    import ctypes
    import torch
    from hexlib_amd import lib as L
    lib = L.load()
    P = ctypes.c_void_p
    a = torch.randn(m, k, dtype=torch.float16, device="cuda")
    wt = torch.randn(n, k, dtype=torch.float16, device="cuda").mul_(0.02)
    bias = torch.zeros(n, dtype=torch.float32, device="cuda")
    out = torch.empty(m, n, dtype=torch.float16, device="cuda")
    call = lambda: lib.matmul_epilogue_f16wt_fp16(P(a.data_ptr()), P(wt.data_ptr()), P(bias.data_ptr()),
                                                  P(out.data_ptr()), m, k, n, act)
    lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
        for _ in range(reps):
            call()
    lib.hexlib_gpu_set_stream(P(torch.cuda.current_stream().cuda_stream))
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e6 / reps)
    del g
    if lib.hexlib_gpu_take_error() != 0:
        raise RuntimeError(f"linear {m}x{k}x{n} reported an error")
    lib.hexlib_gpu_set_stream(P(None))
    return best


def gemm_b32(session, reps: int = 20, library: bool = True) -> list[dict]:
    """The four linears of the cfg-4 product plan at batch 32 (M = 8192), each
    timed in the plan's own buffers as a captured graph of `reps` launches of
    the product op (epilogue included), beside torch.matmul on the same shape
    without an epilogue."""
    from hexlib_amd import encoder as E
    from hexlib_amd.exec.gpu import GpuPlan
    cfg = replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope", batch=32)
    g, _, wb = build_plan(cfg)
    plan = GpuPlan(wb, session)
    rows = []
    try:
        for (spec, ins, (oshape, odt)), (count, idx, op) in unique_ops(g, wb).items():
            if not spec.startswith("matmul_epilogue") or ins[0][0][0] != 32 * cfg.num_tokens:
                continue
            m, k = ins[0][0]
            n = oshape[-1]
            ns = time_blob(session, repeat_op_blob(wb, idx, reps), reps) / reps
            flops = 2.0 * m * k * n
            row = {"op": spec, "shape": [m, k, n], "count": count, "avg_ns": round(ns, 1),
                   "tflops": round(flops / ns / 1e3, 1),
                   "frac": round(flops / ns / 1e3 / MFMA_FP16_PEAK_TFLOPS, 4)}
            if library:
                lns = library_matmul_ns(m, k, n)
                row.update({"library_ns": round(lns, 1), "library_tflops": round(flops / lns / 1e3, 1)})
            if spec != "matmul_epilogue_f16wt":
                pns = plain_linear_ns(m, k, n)
                row.update({"plain_linear_ns": round(pns, 1)})
            rows.append(row)
            log(f"b32 {spec} {m}x{k}x{n}: {ns:.0f} ns ({row['tflops']} TFLOP/s)"
                + (f"; torch.matmul {row['library_ns']:.0f} ns ({row['library_tflops']} TFLOP/s)"
                   if library else ""))
    finally:
        plan.close()
    return rows


# ---- CPU baseline ------------------------------------------------------------------------

def _cpu_images_per_s(cfg, budget_s: float):
    """Images/s of the numpy storage-rounding executor (`oracle.eager.run_stored`,
    the restated `hexlib/exec/interpreter.py:80-205`) on the REFERENCE graph of
    `cfg` (the unfused attention chain the reference builds), for about
    `budget_s` seconds of CPU work."""
    from hexlib_amd import encoder as E
    from hexlib_amd.graph.fuse import fuse
    from oracle import eager
    ref = replace(cfg, attention="unfused")
    g = fuse(E.build_vision_encoder(ref))
    feeds = E.synthetic_feeds(g, ref, seed=0)
    n = 0
    t0 = time.perf_counter()
    while True:
        eager.run_stored(g, feeds)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return n, el


def cpu_per_op(budget_s: float = 0.5) -> list[dict]:
    """Each cfg-2 / cfg-3 op of the cold suite through the oracle's scalar
    kernel restatements (`oracle.kernels`, the reference baselines' numerics)
    on the same inputs: mean ms per call over about `budget_s` seconds."""
    from oracle import kernels as K
    from hexlib_amd.quant import pack_q4_0_nblocked
    rows = []
    for kind, attrs, arrays, out_shape in suite_cases():
        if kind == "rmsnorm":
            fn = lambda: K.rmsnorm_fp16(arrays[0], arrays[1], attrs["eps"])
        elif kind == "layernorm":
            fn = lambda: K.layernorm_fp16(arrays[0], arrays[1], arrays[2], attrs["eps"])
        elif kind == "softmax":
            fn = lambda: K.softmax_fp16(arrays[0])
        elif kind == "rope_2d":
            fn = lambda: K.rope_2d_fp16(*arrays)
        elif kind == "transpose":
            fn = (lambda: K.transpose_th_fp16(arrays[0])) if attrs["perm"] == (1, 0, 2) else \
                 (lambda: K.transpose_hd_fp16(arrays[0]))
        elif kind == "add":
            fn = lambda: K.add_fp16(arrays[0], arrays[1])
        elif kind == "scale":
            fn = lambda: K.scale_fp16(arrays[0], attrs["factor"])
        elif kind == "cast":
            fn = lambda: K.cast_f32_f16(arrays[0])
        elif kind == "patchify":
            fn = lambda: K.patchify_fp32(arrays[0], attrs["patch"], attrs["merge"], attrs["grid_h"], attrs["grid_w"])
        elif kind == "matmul_epilogue":
            act = {"none": 0, "gelu_tanh": 1, "gelu_erf": 2}[attrs["act"]]
            fn = lambda: K.matmul_epilogue_f16w(arrays[0], arrays[1], arrays[2], act)
        elif kind == "matmul":
            fn = lambda: K.matmul_fp16(arrays[0], arrays[1])
        else:
            continue
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s or n >= 1000:
                break
        rows.append({"op": kind, "shape": [list(a.shape) for a in arrays], "ms": round(el / n * 1e3, 3)})
    return rows


def cpu_baseline(cfg, budget_s: float = 12.0) -> dict:
    """The CPU baseline: the reference graph of the headline encoder through
    the numpy executor on this host's cores (the headline figure), plus the
    cfg-1 tiny encoder and the cfg-2 / cfg-3 ops, each timed briefly."""
    from hexlib_amd import encoder as E
    threads = None
    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # noqa: BLE001 -- informational only
        threads = os.cpu_count()
    n, el = _cpu_images_per_s(cfg, budget_s)
    n1, el1 = _cpu_images_per_s(E.TINY_ENCODER, 2.0)
    return {"value": round(n / el, 4), "unit": "images/s", "cores": int(threads or 1),
            "kind": "port",
            "sample": f"{n} image(s) of the cfg-4 256x256 encoder's reference graph (259 ops, unfused "
                      f"attention) through the numpy oracle (storage-rounding interpreter restatement) "
                      f"in {el:.1f} s; os.cpu_count()={os.cpu_count()}, numpy {np.__version__}",
            "cfg1_tiny_encoder_images_per_s": round(n1 / el1, 2),
            "per_op_ms": cpu_per_op()}


def run_variant(session, vcfg, steps: int, label: str) -> dict:
    from hexlib_amd.exec.gpu import GpuPlan
    gv, _, wbv = build_plan(vcfg)
    pv = GpuPlan(wbv, session)
    try:
        s = time_replays(pv, steps, 3)
        out = {"images_per_s": round(steps * vcfg.batch / s, 2),
               "ms_per_step": round(s / steps * 1e3, 3), "batch": vcfg.batch,
               "tokens": vcfg.num_tokens, "steps": steps}
        rows = per_op_in_plan(pv, gv, reps=10)
        mm = [r for r in rows if r["bound"] == "mfma"]
        fl = sum(r["count"] * r["avg_ns"] * r["achieved"] * 1e3 for r in mm)
        t = sum(r["count"] * r["avg_ns"] for r in mm)
        out["gemm_tflops"] = round(fl / t / 1e3, 2) if t else None
        out["gemm_frac_of_peak"] = round(fl / t / 1e3 / MFMA_FP16_PEAK_TFLOPS, 4) if t else None
        out["per_op"] = rows
        log(f"variant {label}: {out['images_per_s']} images/s, GEMMs {out['gemm_tflops']} TFLOP/s")
        for r in rows:
            log(f"  {r['op']:22s} x{r['count']:3d} {r['avg_ns']:9.0f} ns  {r['achieved']:9.2f} {r['unit']:7s} "
                f"({r['frac'] * 100:5.1f}%)  total {r['total_us']:8.1f} us  {r['shape']}")
        return out
    finally:
        pv.close()


# ---- main -------------------------------------------------------------------------------

def main() -> int:
    global FOLD_LN_ROWS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-variants", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="build the plan, launch only the dominant kernel (and, with --copy-ref, a "
                         "plain copy of known size) and print its roofline object")
    ap.add_argument("--copy-ref", action="store_true")
    ap.add_argument("--gemm-b32", action="store_true",
                    help="time the four batch-32 product linears in the plan and torch.matmul on the "
                         "same shapes, print them and exit (the rocprofv3 --pmc target for those GEMMs)")
    ap.add_argument("--no-library", action="store_true", help="with --gemm-b32: skip torch.matmul")
    ap.add_argument("--fold-ln-rows", type=int, default=None,
                    help="fold LayerNorms of at most this many rows into their linear (default: "
                         "fold_rule; 0: every LayerNorm its own launch)")
    ap.add_argument("--plan-only", metavar="VARIANT",
                    choices=("256_b1", "256_b32", "448_b1", "256_b1_q8_0", "256_b1_q4_0"),
                    help="build that plan, time --steps graph replays of it and exit (a rocprofv3 "
                         "target: every kernel of the plan, nothing else)")
    ap.add_argument("--copy-ref-first", action="store_true",
                    help="with --plan-only: first run a plain copy of known size (counter scale)")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print a markdown summary of a rocprofv3 output directory and exit")
    args = ap.parse_args()
    if args.fold_ln_rows is not None:
        FOLD_LN_ROWS = args.fold_ln_rows
    if args.trace_summary:
        print(trace_summary(args.trace_summary))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Images are independent; see DESIGN.md "
              f"for how the plan would shard.", file=sys.stderr)
        return 2

    import torch
    from hexlib_amd import encoder as E
    from hexlib_amd.exec.gpu import GpuPlan, GpuSession

    session = GpuSession()
    if args.plan_only:
        base = replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
        vcfg = {"256_b1": base, "256_b32": replace(base, batch=32),
                "448_b1": replace(E.encoder_at(448), attention="fused_qkv_rope"),
                "256_b1_q8_0": replace(E.QWEN35_VISION_Q8, attention="fused_qkv_rope"),
                "256_b1_q4_0": replace(E.QWEN35_VISION_Q4, attention="fused_qkv_rope")}[args.plan_only]
        if args.copy_ref_first:
            copy_reference()
        _, _, wbv = build_plan(vcfg)
        pv = GpuPlan(wbv, session)
        sec = time_replays(pv, args.steps, args.warmup)
        pv.close()
        session.close()
        print(json.dumps({"plan": args.plan_only, "ops": wbv.n_ops, "steps": args.steps,
                          "ms_per_step": round(sec / args.steps * 1e3, 4),
                          "images_per_s": round(args.steps * vcfg.batch / sec, 2)}))
        return 0
    if args.gemm_b32:
        rows = gemm_b32(session, library=not args.no_library)
        session.close()
        print(json.dumps({"gemm_b32": rows}))
        return 0
    cfg = replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    log("building cfg-4 plan (256x256, batch 1, fused q/k/v linear, q/k rope, fused attention)")
    g, feeds, wb = build_plan(cfg)
    plan = GpuPlan(wb, session)
    if args.roofline_only:
        if args.copy_ref:
            copy_reference()
        roof = roofline(plan, g, cold=False)
        plan.close()
        session.close()
        print(json.dumps({"roofline": roof}))
        return 0
    # first, as in --roofline-only, so the committed rocprof trace of that mode
    # describes the same measurement
    roof = roofline(plan, g)
    sec = time_replays(plan, args.steps, args.warmup)
    ms = sec / args.steps * 1e3
    ips = args.steps * cfg.batch / sec
    log(f"encoder b1: {ms:.3f} ms/image, {ips:.1f} images/s")

    log("per-op timing inside the plan")
    per_op = per_op_in_plan(plan, g)
    for r in per_op:
        log(f"  {r['op']:22s} x{r['count']:3d} {r['avg_ns']:9.0f} ns  {r['achieved']:9.2f} {r['unit']:7s} "
            f"({r['frac'] * 100:5.1f}%)  total {r['total_us']:8.1f} us  {r['shape']}")
    plan_gpu_ns = None
    try:
        from hexlib_amd import lib as L
        rsp = session.invoke(wb.blob, plan.kinds, L.INVOKE_GRAPH | L.INVOKE_TIMED)
        plan_gpu_ns = rsp.cycles_total
    except Exception as e:  # noqa: BLE001
        log(f"timed graph replay failed: {e}")

    share = roof["launches_per_image"] * roof["avg_launch_ns"] / sum(r["count"] * r["avg_ns"] for r in per_op)
    roof["share_of_plan"] = round(share, 3)
    top = per_op[0]
    log(f"roofline: {roof['kernel']} {roof['avg_launch_ns']:.0f} ns/launch, {roof['achieved']} {roof['unit']} "
        f"({roof['frac'] * 100:.2f}% of {roof['bound']} peak), {share * 100:.1f}% of the plan; "
        f"largest in-plan row: {top['op']} {top['shape']} {top['total_us']} us")
    plan.close()

    variants = {}
    if not args.no_variants:
        for label, vcfg, steps in (("256_b32", replace(cfg, batch=32), max(5, args.steps // 10)),
                                   ("448_b1", replace(E.encoder_at(448), attention="fused_qkv_rope"),
                                    max(10, args.steps // 2)),
                                   ("256_b1_reference_graph", E.QWEN35_VISION_FP16, max(10, args.steps // 2)),
                                   ("256_b1_q8_0", replace(E.QWEN35_VISION_Q8, attention="fused_qkv_rope"),
                                    max(10, args.steps // 2)),
                                   ("256_b1_q4_0_reference_config",
                                    replace(E.QWEN35_VISION_Q4, attention="fused_qkv_rope"),
                                    max(10, args.steps // 2))):
            log(f"variant {label}")
            try:
                variants[label] = run_variant(session, vcfg, steps, label)
            except Exception as e:  # noqa: BLE001 -- a variant failure must not lose the headline line
                log(f"variant {label} failed: {type(e).__name__}: {e}")
                variants[label] = {"error": f"{type(e).__name__}: {e}"}

    suite_rows = [] if args.no_suite else suite(session)
    q4_rows = [] if args.no_suite else q4_gemm_sweep()
    q4n_rows = [] if args.no_suite else q4n_gemm_rows()

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (numpy oracle)")
        cpu = cpu_baseline(cfg)

    line = {
        "metric": METRIC, "value": round(ips, 2), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: seeded U[0,1] image, N(0,0.02) fp16 weights, random init",
        "config": {"workload": "vit_encoder_256_b1 (BASELINE cfg 4: 12 blocks, hidden 768, "
                               "12 heads, MLP 3072, LayerNorm, 2D RoPE, merger; per block one q/k/v linear "
                               "with the q/k rope in its epilogue, one fused attention op, the residual adds "
                               f"in the linears' epilogues; {wb.n_ops} ops as one hipGraph)",
                   "image": 256, "batch": 1, "tokens": 256, "attention": cfg.attention,
                   "plan_ops": wb.n_ops, "plan_gpu_ns": plan_gpu_ns},
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_op_in_plan": per_op,
        "per_op_suite_cold": suite_rows,
        "q4_gemm_cfg5": q4_rows,
        "q4_0_reference_abi_gemm": q4n_rows,
        "variants": variants,
    }
    session.close()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
