"""Writes the committed whole-plan artefact and its expected output:

* `tiny_encoder.hxplan` -- the BASELINE cfg-1 encoder (TINY_ENCODER, seeded
  synthetic weights and image, seed 0) as a plan file with its sample image;
* `tiny_encoder_out.npy` -- the storage-rounding oracle's output for the same
  graph and feeds (`oracle.eager.run_stored` of the fused graph).

Run from the repository root: `python tests/golden/make_tiny_plan.py`.
`tests/test_planfile.py` checks that both files are current.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from hexlib_amd import encoder as E  # noqa: E402
from hexlib_amd.exec import planfile  # noqa: E402
from hexlib_amd.exec.wholeplan import build_whole_plan_batch  # noqa: E402
from hexlib_amd.graph.fuse import fuse  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
PLAN = os.path.join(HERE, "tiny_encoder.hxplan")
EXPECTED = os.path.join(HERE, "tiny_encoder_out.npy")


def build():
    cfg = E.TINY_ENCODER
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=0)
    return g, feeds, build_whole_plan_batch(g, feeds)


def expected(g, feeds):
    from oracle import eager
    f = fuse(g)
    return eager.run_stored(f, feeds)[g.outputs[0]].astype(np.float16)


def main():
    g, feeds, wb = build()
    planfile.save(wb, PLAN)
    np.save(EXPECTED, expected(g, feeds), allow_pickle=False)
    print(f"wrote {PLAN} ({os.path.getsize(PLAN)} B) and {EXPECTED}")


if __name__ == "__main__":
    main()
