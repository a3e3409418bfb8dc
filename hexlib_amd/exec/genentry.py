"""Generate the C++ entry adapters and the kind table from `runner.SPECS`.

The reference generates one `int <k>_entry(const hexlib_args *)` per kernel
and `hexlib_kernel_table[]` from its RunnerSpec table
(`hexlib/runtime/genentry.py:131-373`), so the argument mapping is declared
once. Same here; every entry:

1. checks the buffer count and that no buffer is NULL (ERR_INVAL_PARAMS);
2. checks EVERY buffer's declared dtype and layout against the spec
   (ERR_REQUIRES) -- a wrongly typed buffer would otherwise be read at the
   wrong stride;
3. derives the scalars from the tensors' own extents (`numel:`, `dim:`,
   `rows:`) or from op params (`attr:`, floats as IEEE bits);
4. refuses (ERR_INVAL_PARAMS) any buffer smaller than the extent the kernel
   will touch, and non-positive dimensions -- so a malformed blob can never
   become an out-of-bounds GPU access;
5. calls the kernel_api function and reports a failed launch as ERR_INTERNAL.

`python -m hexlib_amd.exec.genentry` rewrites `hexlib_amd/csrc/gen_entries.cpp`;
the build does this before compiling and a CPU test checks the committed file
is current.
"""
from __future__ import annotations

import os
import re
import sys

from hexlib_amd.exec.runner import KIND_ID, SPECS, WIRE_RAW, RunnerSpec
from hexlib_amd.exec.wire import DTYPE_ID, LAYOUT_ID

_CTYPE = {"fp16": "hexlib_hf", "fp32": "float", "int32": "int"}
OUT_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "csrc", "gen_entries.cpp")


_NAME = re.compile(r"[A-Za-z_][A-Za-z0-9_]*|[0-9]+")


def _top_level_factors(ext: str) -> list[str]:
    out, depth, cur = [], 0, ""
    for ch in ext:
        depth += ch == "("
        depth -= ch == ")"
        if ch == "*" and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    out.append(cur.strip())
    return out


def _wide(ext: str) -> str:
    """An extent (a product of scalars, literals and parenthesised
    multiply-free int expressions, optionally written with a leading
    `(uint64_t)` cast) as a saturating 128-bit product: each factor is widened
    before it is multiplied and a product that would pass 2^128 saturates, so
    the comparison against a buffer's element count can never wrap."""
    factors = _top_level_factors(ext.replace("(uint64_t)", ""))
    for f in factors:
        if not (_NAME.fullmatch(f) or (f.startswith("(") and f.endswith(")") and "*" not in f)):
            raise ValueError(f"extent {ext!r}: factor {f!r} is not a name, a literal or a "
                             f"multiply-free parenthesised expression")
    expr = f"(hx_u128) {factors[0]}"
    for f in factors[1:]:
        expr = f"hx_mul_sat({expr}, (hx_u128) {f})"
    return expr


def _scalar_expr(src: str, ctype: str, param_index: int) -> str:
    kind, _, rest = src.partition(":")
    if kind == "attr":
        return f"((const {ctype} *) a->params)[{param_index}]"
    if kind == "numel":
        return f"hx_numel(a, {int(rest)})"
    i, axis = (int(v) for v in rest.split(":"))
    if kind == "dim":
        return f"(uint64_t) a->ne[{i}][{axis}]"
    if kind == "rows":
        return f"(a->ne[{i}][{axis}] ? hx_numel(a, {i}) / a->ne[{i}][{axis}] : 0)"
    raise ValueError(f"unknown scalar source {src!r}")


def emit_entry(name: str, spec: RunnerSpec) -> str:
    n_in = len(spec.inputs)
    n_buf = n_in + 1
    dtypes = list(spec.inputs) + [spec.out_dtype]
    layouts = spec.buf_layouts()
    lines = [f"int {spec.entry}_entry(const hexlib_args *a) {{",
             f"    /* KIND_ID {KIND_ID[name]} ({name!r}): {spec.kind} -> {spec.entry} */",
             f"    if (a->n_buf != {n_buf}) return HEXLIB_DSP_ERR_INVAL_PARAMS;"]
    for i in range(n_buf):
        lines.append(f"    if (!a->buf[{i}]) return HEXLIB_DSP_ERR_INVAL_PARAMS;")
    for i, dt in enumerate(dtypes):
        lines.append(f"    if (a->dtype[{i}] != {DTYPE_ID[dt]}u) return HEXLIB_DSP_ERR_REQUIRES;"
                     f"  /* {dt} */")
    for i, lay in enumerate(layouts):
        lines.append(f"    if (a->layout[{i}] != {LAYOUT_ID[lay]}u) return HEXLIB_DSP_ERR_REQUIRES;"
                     f"  /* {lay} */")
    param_index = 0
    args_scalar = []
    for sc in spec.scalars:
        if sc.source.startswith("attr:"):
            expr = _scalar_expr(sc.source, sc.ctype, param_index)
            param_index += 1
            if sc.ctype == "float":
                lines.append(f"    const float {sc.name} = {expr};")
            else:
                lines.append(f"    const int {sc.name} = {expr};")
                if sc.codes:
                    codes = sorted(v for _, v in sc.codes)
                    lines.append(f"    if ({sc.name} < {codes[0]} || {sc.name} > {codes[-1]}) "
                                 f"return HEXLIB_DSP_ERR_INVAL_PARAMS;")
                elif sc.default is not None:
                    lines.append(f"    if ({sc.name} < 0) return HEXLIB_DSP_ERR_INVAL_PARAMS;")
                else:
                    lines.append(f"    if ({sc.name} <= 0) return HEXLIB_DSP_ERR_INVAL_PARAMS;")
        else:
            expr = _scalar_expr(sc.source, sc.ctype, param_index)
            lines.append(f"    const hx_u128 {sc.name}_u = {expr};")
            lines.append(f"    if ({sc.name}_u == 0 || {sc.name}_u > 0x7fffffffu) "
                         f"return HEXLIB_DSP_ERR_INVAL_PARAMS;")
            lines.append(f"    const int {sc.name} = (int) {sc.name}_u;")
        args_scalar.append(sc.name)
    for i, ext in enumerate(spec.extents):
        lines.append(f"    if ({_wide(ext)} > hx_numel(a, {i})) "
                     f"return HEXLIB_DSP_ERR_INVAL_PARAMS;")
    for cond in spec.checks:
        lines.append(f"    if (!({cond})) return HEXLIB_DSP_ERR_INVAL_PARAMS;")
    bufs = []
    for i, dt in enumerate(spec.inputs):
        ctype = "unsigned char" if dt in WIRE_RAW else _CTYPE[dt]
        bufs.append(f"(const {ctype} *) a->buf[{i}]")
    bufs.append(f"({_CTYPE[spec.out_dtype]} *) a->buf[{n_in}]")
    call = ", ".join(bufs + args_scalar)
    lines.append(f"    {spec.entry}({call});")
    lines.append("    return hx_entry_status();")
    lines.append("}")
    return "\n".join(lines)


def generate() -> str:
    parts = [
        "// GENERATED by hexlib_amd/exec/genentry.py from hexlib_amd/exec/runner.py SPECS.",
        "// Do not edit: run `python -m hexlib_amd.exec.genentry`.",
        '#include <stdint.h>',
        '',
        '#include "hexlib_gpu.h"',
        '#include "internal.h"',
        '',
        'namespace {',
        'typedef unsigned __int128 hx_u128;',
        '// Element count of buffer i: four uint32 factors, widened before each',
        '// multiply, so the product (< 2^128) never wraps.',
        'inline hx_u128 hx_numel(const hexlib_args *a, int i) {',
        '    return (hx_u128) a->ne[i][0] * a->ne[i][1] * a->ne[i][2] * a->ne[i][3];',
        '}',
        '// a * b, or the largest value where the product would pass 2^128.',
        'inline hx_u128 hx_mul_sat(hx_u128 a, hx_u128 b) {',
        '    hx_u128 r;',
        '    return __builtin_mul_overflow(a, b, &r) ? ~(hx_u128) 0 : r;',
        '}',
        '// A launch error recorded while running an entry is an op failure.',
        'inline int hx_entry_status() {',
        '    if (hx::dry_run()) return HEXLIB_DSP_OK;',
        '    const int e = hexlib_gpu_take_error();',
        '    if (e != 0) { hx::note((hipError_t) e); return HEXLIB_DSP_ERR_INTERNAL; }',
        '    return HEXLIB_DSP_OK;',
        '}',
        '}  // namespace',
        '',
        'extern "C" {',
        '',
    ]
    for name, spec in SPECS.items():
        parts.append(emit_entry(name, spec))
        parts.append("")
    parts.append("const struct hexlib_kernel_entry hexlib_kernel_table[] = {")
    for name in sorted(SPECS, key=lambda n: KIND_ID[n]):
        parts.append(f'    {{{KIND_ID[name]}u, "{name}", {SPECS[name].entry}_entry}},')
    parts.append("};")
    parts.append("const uint32_t hexlib_kernel_table_len =")
    parts.append("    sizeof(hexlib_kernel_table) / sizeof(hexlib_kernel_table[0]);")
    parts.append("")
    parts.append('}  // extern "C"')
    parts.append("")
    return "\n".join(parts)


def write(path: str = OUT_PATH) -> str:
    text = generate()
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return path


if __name__ == "__main__":
    print(write(sys.argv[1] if len(sys.argv) > 1 else OUT_PATH))
