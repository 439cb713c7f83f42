"""Pins of the oracle's split-KV grouped-query decode attention
(16 query heads, 2 KV heads, head_dim 128)."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle.reference import compare_values, gqa_f64
from tests import _kat

F = np.float32
SCALE = 1.0 / math.sqrt(128.0)


def test_reference_gqa_smoke_fixture():
    q, k, v, tol = _kat.gqa_smoke_case(37)
    got = O.f16_to_f32(O.gqa(q, k, v, 37, dtype="f16"))
    want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), 37, SCALE)
    assert np.abs(got - want).max() <= tol


def test_reference_gqa_workspace_fixture():
    q, k, v, lens, tol = _kat.gqa_workspace_case()
    for kv_len in lens:
        got = O.f16_to_f32(O.gqa(q, k, v, kv_len, dtype="f16"))
        want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), kv_len, SCALE)
        assert np.abs(got - want).max() <= tol, kv_len


@pytest.mark.parametrize("kv_len", [1, 7, 128, 512, 585, 1024, 2048])
def test_random_inputs_at_the_correctness_tool_lengths(kv_len):
    # tools/correctness/run_qwen2_gqa_check.py:41-47,94-99: seed 20260824, atol = rtol = 3.5e-3
    rng = np.random.default_rng([20260824, kv_len])
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), kv_len, SCALE)
    # bf16 output: the comparison tolerance of the tool widened to bf16 rounding
    result = compare_values(got.tolist(), want.tolist(), atol=3.5e-3, rtol=2.0 ** -8)
    assert result["passed"], result


def test_single_token_returns_the_value_row_exactly():
    rng = np.random.default_rng(2)
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, 64, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, 64, 128)).astype(F))
    out = O.gqa(q, k, v, 1).reshape(16, 128)
    for h in range(16):
        assert out[h].tobytes() == v[h // 8, 0].tobytes()


def test_identical_keys_average_the_values():
    rng = np.random.default_rng(4)
    kv_len = 300
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    row = O.f32_to_bf16(rng.standard_normal(128).astype(F))
    k = np.broadcast_to(row, (2, kv_len, 128)).copy()
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    out = O.bf16_to_f32(O.gqa(q, k, v, kv_len)).reshape(16, 128)
    mean = O.bf16_to_f32(v).astype(np.float64)[:, :kv_len].mean(axis=1)
    for h in range(16):
        assert np.all(np.abs(out[h] - mean[h // 8]) <= 2.0 ** -8 * np.abs(mean[h // 8]) + 1e-5)


@pytest.mark.parametrize("chunk", [128, 256, 512, 1024])
def test_split_size_changes_only_rounding(chunk):
    rng = np.random.default_rng(6)
    kv_len = 2000
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, 2048, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, 2048, 128)).astype(F))
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len, chunk=chunk, mid_max=0))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), kv_len, SCALE)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 2e-4)


def test_planted_wrong_group_mapping_fails():
    """Feeding the KV heads swapped is what an oracle with group = h % 2 would see."""

    q, k, v, tol = _kat.gqa_smoke_case(37)
    got = O.f16_to_f32(O.gqa(q, k[::-1].copy(), v[::-1].copy(), 37, dtype="f16"))
    want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), 37, SCALE)
    assert np.abs(got - want).max() > tol


def test_split_plan_covers_every_regime():
    # (chunk, flat_max, mid_max, max_splits): flat path with 32-token splits up
    # to 32 x 32 tokens (8 x 32 with the reference's 16 x 8 x 130 workspace),
    # round path with 128-token splits up to 8192 tokens, 256-token beyond
    assert O.gqa_plan(2048) == (256, 1024, 2048, 32)
    assert O.gqa_plan(32768) == (256, 1024, 8192, 128)
    assert O.gqa_plan(65536) == (256, 1024, 8192, 256)
    assert O.gqa_plan(100) == (256, 100, 100, 4)
    assert O.gqa_plan(512, split_limit=8) == (256, 256, 512, 8)
    assert O.gqa_plan(1) == (256, 1, 1, 1)
    # a capped workspace also caps the long splits' count
    chunk, _, mid_max, splits = O.gqa_plan(32768, split_limit=8)
    assert splits == 8 and chunk * 8 >= 32768 and mid_max == 1024


@pytest.mark.parametrize("kv_len", [31, 32, 33, 200, 1023, 1024, 1025, 1087, 2047, 2048, 2049, 2100])
def test_flat_path_boundaries_match_fp64(kv_len):
    """Split edges of the flat path (a full split, a one-token split, the
    32-split maximum), of its two-token-per-group form (64-token splits up to
    2048 tokens) and the first lengths past it (round path, 128-token
    splits)."""

    rng = np.random.default_rng([7, kv_len])
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, 2100, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, 2100, 128)).astype(F))
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), kv_len, SCALE)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 2e-4)


@pytest.mark.parametrize("kv_len", [1, 7, 64, 128, 512])
@pytest.mark.parametrize("regime", [dict(flat_max=0), dict(flat_max=0, mid_max=0)])
def test_round_path_at_short_lengths_matches_the_workspace_fixture(kv_len, regime):
    """flat_max=0 forces the round path with 128-token splits (what a capped
    workspace uses past its flat limit), mid_max=0 too its 256-token splits;
    the reference fixture's tolerance holds for both."""

    q, k, v, lens, tol = _kat.gqa_workspace_case()
    got = O.f16_to_f32(O.gqa(q, k, v, kv_len, dtype="f16", **regime))
    want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), kv_len, SCALE)
    assert np.abs(got - want).max() <= tol


def test_flat_and_round_paths_agree():
    rng = np.random.default_rng(9)
    kv_len = 300
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    flat = O.bf16_to_f32(O.gqa(q, k, v, kv_len))
    rnd = O.bf16_to_f32(O.gqa(q, k, v, kv_len, flat_max=0))
    # different fp32 operation orders, the same attention to bf16 rounding
    assert np.all(np.abs(flat - rnd) <= 2.0 ** -7 * np.abs(rnd) + 1e-4)


def test_planted_dropped_flat_split_fails():
    """An oracle that lost the last (one-token) split of the flat path is
    caught by the fp64 check: at kv_len 33 the dropped token is the one with
    a dominant key."""

    rng = np.random.default_rng(11)
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = rng.standard_normal((2, 33, 128)).astype(F)
    k[:, 32] = 4.0 * np.sign(O.bf16_to_f32(q).reshape(2, 8, 128).mean(axis=1))
    k = O.f32_to_bf16(k)
    v = O.f32_to_bf16(rng.standard_normal((2, 33, 128)).astype(F))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), 33, SCALE)
    good = O.bf16_to_f32(O.gqa(q, k, v, 33))
    dropped = O.bf16_to_f32(O.gqa(q, k[:, :32].copy(), v[:, :32].copy(), 32))
    assert np.all(np.abs(good - want) <= 2.0 ** -8 * np.abs(want) + 2e-4)
    assert np.abs(dropped - want).max() > 0.1
