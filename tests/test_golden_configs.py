"""The committed config fixtures (tests/golden/configs.json) are what the pinned
oracle computes on the seeded inputs of the five workload configurations, and
the chunked weight generator the GPU tests use draws exactly the same numbers."""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_fixtures  # noqa: E402
from kv260gemv import configs as cf  # noqa: E402

FIXTURES = os.path.join(HERE, "golden", "configs.json")


def test_chunked_weights_equal_whole_matrix():
    m = cf.Matrix("t", 1000, 512, 5, 6)
    whole = cf.weights(m)
    for rows_per_chunk in (1, 128, 999, 4096):
        parts = np.concatenate([w for _, w in cf.weight_chunks(m, rows_per_chunk)])
        assert np.array_equal(whole, parts)


def test_config_shapes_and_bytes():
    chain = cf.decode_chain()
    assert len(chain) == 65
    assert cf.chain_weight_bytes() == 695_107_584          # docs/buildlog/0013-release-session.md:131-132
    assert cf.chain_algorithmic_bytes() == 697_388_288
    assert cf.O_PROJ.algorithmic_bytes == 2_369_792
    assert cf.LM_HEAD.weight_bytes == 147_750_912
    assert [m.rows for m in cf.LAYER_SHAPES] == [3072, 2048, 16384, 2048]


def test_fixtures_reproduce_from_the_oracle():
    """All five configurations recomputed by the oracle (about a minute)."""
    with open(FIXTURES) as f:
        committed = json.load(f)
    assert make_fixtures.build() == committed


def test_gen_vectors_reproduce_from_the_oracle():
    """The reference's exactness cases (gen_vectors.py, one default_rng(4) stream)
    recomputed by both oracle implementations match the committed digests."""
    import make_gen_vectors
    with open(os.path.join(HERE, "golden", "gen_vectors.json")) as f:
        committed = json.load(f)
    assert make_gen_vectors.build() == committed
    assert [c["name"] for c in committed["cases"]][:5] == ["k256_n16", "k2048_n64", "k8192_n16", "k256_n32", "k8192_n32"]
