"""TEST INFRASTRUCTURE ONLY -- the CPU checker for hexlib_amd's GPU path.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
may import anything here, and only to CHECK or to time the CPU baseline. No
product code path (hexlib_amd) imports this package; the GPU path fails loudly
when its HIP library is missing rather than falling back to anything here.

Contents, each citing the reference file it restates:

* `refs`     -- the op registry's numpy references
                (`hexlib/graph/opdefs/elementwise.py:40-156`, `fused.py:44-53`,
                `structural.py:55-254`), plus `rmsnorm` from
                `kernels/rmsnorm_fp16/baseline.c:6-19`.
* `eager`    -- `run_fp32`, the fp32 eager oracle (`hexlib/graph/eager.py:32-132`),
                and `run_stored`, the storage-rounding plan executor
                (`hexlib/exec/interpreter.py:80-205` with `hexlib/exec/vtcm.py:90-146`):
                fp32 compute, every op output rounded to its declared storage dtype.
* `kernels`  -- per-kernel scalar contracts (`kernels/*/baseline.c` +
                `kernel_api.h`), vectorised in numpy, used by the per-op GPU parity
                tests.
* `quant`    -- q4_0 scalar transcription + dequantizer (`hexlib/exec/quant.py:62-135`,
                llama.cpp `quantize_row_q4_0_ref` / `dequantize_row_q4_0`).
* `ref`      -- ctypes access to `oracle/_ref/libhexlib_ref.so`, the reference's
                own `kernels/*/baseline.c` compiled from `/root/reference` by
                `oracle/Makefile`; used to pin `kernels` above.

Parity-pinning status per function is recorded in each module's docstring.
"""
