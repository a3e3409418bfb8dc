"""The oracle against the committed upstream golden vectors.

Restates the reference's gate (`hexlib/tests/test_vision_oracle.py:39-150`,
`test_exec_interpreter.py:57-79`): the fp32 eager oracle must reproduce the
upstream model's merged output, patchify must reproduce upstream's literal
permute chain, a wrong epsilon must be caught, and the storage-rounding
executor must stay within 1e-3 relative of upstream while being measurably
worse than fp32.
"""
import os

import numpy as np

from hexlib_amd import encoder as E
from hexlib_amd.graph.fuse import fuse
from oracle import eager, refs
from tests.conftest import GOLDEN


def _feeds(graph, cfg, z):
    feeds = E.feeds_from_params(graph, cfg, lambda n: z["param::" + n])
    feeds["image"] = z["image"]
    return feeds


def test_golden_file_is_present_and_complete(golden):
    assert os.path.getsize(GOLDEN) > 1024
    for key in ("image", "patches", "patches_upstream", "expected_merged", "expected_last_hidden"):
        assert key in golden.files
    assert any(k.startswith("param::") for k in golden.files)


def test_learned_pos_grid_differs_from_patch_grid(golden):
    # Otherwise the bilinear weights are all 0/1 and the resample is untested.
    side = int(golden["param::pos_embed.weight"].shape[0] ** 0.5)
    assert side != E.GOLDEN_TINY.grid
    pos = np.linspace(0, side - 1, E.GOLDEN_TINY.grid)
    assert np.count_nonzero(pos - pos.astype(np.int64)) > 0


def test_patchify_matches_upstream_permute_chain(golden):
    cfg = E.GOLDEN_TINY
    (out,) = refs.patchify((golden["image"],), {
        "patch": cfg.patch_size, "temporal_patch": cfg.temporal_patch_size,
        "merge": cfg.spatial_merge_size, "grid_h": cfg.grid, "grid_w": cfg.grid})
    np.testing.assert_array_equal(out, golden["patches_upstream"])


def test_encoder_matches_upstream(golden):
    cfg = E.GOLDEN_TINY
    g = E.build_vision_encoder(cfg)
    out = eager.run_fp32(g, _feeds(g, cfg, golden))[g.outputs[0]]
    np.testing.assert_allclose(out, golden["expected_merged"], rtol=1e-4, atol=1e-5)


def test_fusion_does_not_change_the_answer(golden):
    cfg = E.GOLDEN_TINY
    g = E.build_vision_encoder(cfg)
    feeds = _feeds(g, cfg, golden)
    a = eager.run_fp32(g, feeds)[g.outputs[0]]
    b = eager.run_fp32(fuse(g), feeds)[g.outputs[0]]
    np.testing.assert_array_equal(a, b)


def test_a_wrong_epsilon_is_caught(golden):
    from dataclasses import replace

    cfg = replace(E.GOLDEN_TINY, layernorm_eps=1e-1)
    g = E.build_vision_encoder(cfg)
    out = eager.run_fp32(g, _feeds(g, cfg, golden))[g.outputs[0]]
    assert not np.allclose(out, golden["expected_merged"], rtol=1e-4, atol=1e-5)


def test_stored_fp16_executor_is_close_but_worse(golden):
    from dataclasses import replace

    cfg = replace(E.GOLDEN_TINY, act_dtype="fp16")
    g = fuse(E.build_vision_encoder(cfg))
    feeds = _feeds(g, cfg, golden)
    want = golden["expected_merged"]
    got16 = eager.run_stored(g, feeds)[g.outputs[0]]
    got32 = eager.run_fp32(g, feeds)[g.outputs[0]]
    rel16 = np.abs(got16 - want).max() / np.abs(want).max()
    rel32 = np.abs(got32 - want).max() / np.abs(want).max()
    assert rel16 < 1e-3
    assert rel32 < rel16


def test_rope_tables_match_upstream_inv_freq(golden):
    cfg = E.GOLDEN_TINY
    half = cfg.head_dim // 2
    inv = 1.0 / cfg.rope_theta ** (np.arange(0, half, 2, dtype=np.float64) / half)
    np.testing.assert_allclose(inv, golden["buffer::rotary_pos_emb.inv_freq"], rtol=1e-6)
    cos, sin = E.rope_tables(cfg)
    assert cos.shape == (cfg.num_tokens, cfg.head_dim)
    np.testing.assert_allclose(cos * cos + sin * sin, 1.0, atol=1e-6)
