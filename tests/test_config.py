"""Host logic without a GPU: the runtime's config validation, score words and boundary budgets
agree with the oracle's (R:625-637 for the reference's keys; the block policies' keys have no
reference counterpart)."""
from types import SimpleNamespace

import pytest

import oracle as O

REQ = SimpleNamespace(rid="r", session=None)
BASE = {"budget": 2048, "prefix": 128, "recent": 512, "seed": 0}
CONFIGS = [
    {"name": "head_sum_2048"},
    {"name": "head_sum_2048", "score_delay": 9},  # ignored: not a block policy
    {"name": "prefix_sliding_2048", "budget": 640},
    {"name": "prefix_sliding_2048"},  # B != P + R
    {"name": "block_sum_2048"},
    {"name": "block_max_2048", "block": 4, "score_delay": 128, "max_evicted_blocks": 512},
    {"name": "block_sum_2048", "score_delay": 512},
    {"name": "block_sum_2048", "score_delay": 513},  # past the recent window
    {"name": "block_sum_2048", "score_delay": -1},
    {"name": "block_sum_2048", "max_evicted_blocks": True},
    {"name": "block_sum_2048", "max_evicted_blocks": 2.0},
    {"name": "block_sum_2048", "block": 3},
    {"name": "block_max_2048", "block": 4, "score_delay": 128, "max_evicted_blocks": 512,
     "block_score": "step_max"},  # the report's counters (score kind 4)
    {"name": "block_sum_2048", "block": 64, "block_score": "step_max"},
    {"name": "block_sum_2048", "block": 128, "block_score": "step_max"},  # blocks of at most 64
    {"name": "block_sum_2048", "shared": False, "block_score": "step_max"},  # counters are per layer
    {"name": "block_sum_2048", "block_score": "position"},
    {"name": "block_sum_2048", "block_score": "mean"},
    {"name": "head_sum_2048", "block_score": "mean"},  # ignored: not a block policy
    {"name": "nope_2048"},
]


@pytest.fixture
def requests():
    from gstar_evict import requests as R
    return R


@pytest.mark.parametrize("extra", CONFIGS)
def test_validation_matches_the_oracle(requests, extra):
    cfg = {**BASE, **extra}
    got, want = requests.live_entry(REQ, cfg, "live"), O.live_entry(cfg)
    assert (got["error"] is None) == (want["error"] is None), cfg
    assert got["mode"] == want["mode"]


def test_score_word_carries_the_delay(requests):
    e = requests.live_entry(REQ, {**BASE, "name": "block_max_2048", "block": 4, "score_delay": 128}, "live")
    assert requests.score_word(e) == 2 | 128 << requests.SCORE_DELAY_SHIFT
    assert requests.score_word(requests.live_entry(REQ, {**BASE, "name": "head_sum_2048"}, "live")) == 1
    assert requests.score_word(requests.live_entry(REQ, {**BASE, "name": "random_2048"}, "live")) == 3
    bad = requests.live_entry(REQ, {**BASE, "name": "block_sum_2048", "score_delay": 999}, "live")
    assert requests.score_word(bad) == 0


def test_score_word_of_block_counters(requests):
    """Kind 4 with log2(block) in bits 4-7 and the delay from bit 8."""
    cfg = {**BASE, "name": "block_sum_2048", "block": 16, "score_delay": 100, "block_score": "step_max"}
    assert requests.score_word(requests.live_entry(REQ, cfg, "live")) == 4 | 4 << 4 | 100 << 8
    cfg = {**BASE, "name": "block_max_2048", "block": 1, "block_score": "step_max"}
    assert requests.score_word(requests.live_entry(REQ, cfg, "live")) == 4


def test_boundary_budget_caps_the_evicted_blocks(requests):
    cfg = {**BASE, "name": "block_sum_2048", "block": 16, "max_evicted_blocks": 64}
    assert requests.boundary_budget(cfg, 4096) == 4096 - 64 * 16
    assert requests.boundary_budget(cfg, 2100) == 2048  # the cap does not bind
    assert requests.boundary_budget({**BASE, "name": "head_sum_2048", "max_evicted_blocks": 1}, 4096) == 2048
