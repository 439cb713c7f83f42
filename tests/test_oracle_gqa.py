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


@pytest.mark.parametrize("split_cap", [1, 2, 4, 16, 63])
def test_split_size_changes_only_rounding(split_cap):
    """Caps 1..63 at 2000 tokens give splits of 63, 32, 16, 4 and 1 rounds
    (one split of every token, down to 32-token splits); each is the same
    attention up to fp32 rounding."""

    rng = np.random.default_rng(6)
    kv_len = 2000
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, 2048, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, 2048, 128)).astype(F))
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len, split_cap=split_cap))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), kv_len, SCALE)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 2e-4)


def test_planted_wrong_group_mapping_fails():
    """Feeding the KV heads swapped is what an oracle with group = h % 2 would see."""

    q, k, v, tol = _kat.gqa_smoke_case(37)
    got = O.f16_to_f32(O.gqa(q, k[::-1].copy(), v[::-1].copy(), 37, dtype="f16"))
    want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), 37, SCALE)
    assert np.abs(got - want).max() > tol


def test_split_plan():
    # (split_cap, max_splits): up to 256 splits per KV head, 32-token rounds;
    # a caller-sized workspace caps the splits
    assert O.gqa_plan(2048) == (256, 64)
    assert O.gqa_plan(32768) == (256, 256)
    assert O.gqa_plan(65536) == (256, 256)
    assert O.gqa_plan(100) == (256, 4)
    assert O.gqa_plan(512, split_limit=8) == (8, 8)
    assert O.gqa_plan(1) == (256, 1)
    assert O.gqa_plan(2048, split_limit=O.GQA_STEP_SPLITS) == (32, 32)
    # one-round splits up to 256 rounds, then the fewest rounds per split
    assert [O.gqa_split_tokens(n, 256) for n in (1, 8192, 8193, 16384, 16385, 32768, 65536)] == \
        [32, 32, 64, 64, 96, 128, 256]
    # the decode step: one round per split up to 1024 tokens
    assert [O.gqa_split_tokens(n, 32) for n in (1024, 1025, 2048, 2049)] == [32, 64, 64, 96]


@pytest.mark.parametrize("cap", [1, 3, 8, 32, 256])
def test_split_rule_is_the_fewest_whole_rounds_within_the_cap(cap):
    for n in range(1, 9000, 7):
        c = O.gqa_split_tokens(n, cap)
        assert c % 32 == 0 and -(-n // c) <= cap, (n, c)
        assert c == 32 or -(-n // (c - 32)) > cap, (n, c)  # one round fewer breaks the cap


@pytest.mark.parametrize("split_cap", [None, O.GQA_STEP_SPLITS, 3])
@pytest.mark.parametrize("kv_len", [31, 32, 33, 200, 1023, 1024, 1025, 1087, 2047, 2048, 2049, 2100])
def test_split_edges_match_fp64(kv_len, split_cap):
    """Round and split edges (a full round, a one-token round, 16 / 17 splits
    on either side of a merge group, the decode step's one-round limit at
    1024 tokens and its two-round splits past it, splits of many rounds with
    cap 3)."""

    rng = np.random.default_rng([7, kv_len])
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, 2100, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, 2100, 128)).astype(F))
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len, split_cap=split_cap))
    want = gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v), kv_len, SCALE)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 2e-4)


@pytest.mark.parametrize("kv_len", [1, 7, 64, 128, 512])
@pytest.mark.parametrize("split_cap", [1, 2])
def test_many_round_splits_match_the_workspace_fixture(kv_len, split_cap):
    """Caps of one and two splits make every length past a round a split of
    several rounds (the online rescale between rounds); the reference
    fixture's tolerance holds."""

    q, k, v, lens, tol = _kat.gqa_workspace_case()
    got = O.f16_to_f32(O.gqa(q, k, v, kv_len, dtype="f16", split_cap=split_cap))
    want = gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), kv_len, SCALE)
    assert np.abs(got - want).max() <= tol


def test_one_round_and_many_round_splits_agree():
    rng = np.random.default_rng(9)
    kv_len = 300
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    k = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    flat = O.bf16_to_f32(O.gqa(q, k, v, kv_len))
    one = O.bf16_to_f32(O.gqa(q, k, v, kv_len, split_cap=1))
    # different fp32 operation orders, the same attention to bf16 rounding
    assert np.all(np.abs(flat - one) <= 2.0 ** -7 * np.abs(one) + 1e-4)


def test_planted_missing_rescale_fails():
    """The rescale between rounds matters: a cache whose later rounds hold
    the dominant keys, read as one split of 10 rounds, differs from the
    fp64 attention by far more than rounding if the earlier rounds' sums are
    not scaled down.  Summing each round's softmax separately (what a dropped
    rescale amounts to, restated here in fp64) fails; the oracle passes."""

    rng = np.random.default_rng(12)
    kv_len = 320
    q32 = rng.standard_normal(2048).astype(F)
    k32 = rng.standard_normal((2, kv_len, 128)).astype(F)
    k32[:, 288:] += 3.0 * np.sign(q32.reshape(2, 8, 128).mean(axis=1))[:, None, :]
    q, k = O.f32_to_bf16(q32), O.f32_to_bf16(k32)
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(F))
    qf, kf, vf = O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(v)
    want = gqa_f64(qf, kf, vf, kv_len, SCALE)
    got = O.bf16_to_f32(O.gqa(q, k, v, kv_len, split_cap=1))
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 2e-4)
    s = np.einsum("gtd,ghd->ght", kf.astype(np.float64), qf.reshape(2, 8, 128).astype(np.float64)) * SCALE
    wrong = np.zeros((2, 8, 128))
    norm = np.zeros((2, 8, 1))
    for r0 in range(0, kv_len, 32):
        w = np.exp(s[:, :, r0:r0 + 32] - s[:, :, r0:r0 + 32].max(axis=2, keepdims=True))
        wrong += np.einsum("ght,gtd->ghd", w, vf[:, r0:r0 + 32].astype(np.float64))
        norm += w.sum(axis=2, keepdims=True)
    assert np.abs((wrong / norm).reshape(-1) - want.reshape(-1)).max() > 0.05


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
