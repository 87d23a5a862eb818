"""Pins the oracle's device summation order (oracle.dit_order(DIT_ORDER_DEVICE)), the mode
that restates the f32 sums of the library's batch-1 DiT kernels so that the flow head can be
compared bit for bit.

- exp_rep (the e^x both sides evaluate from correctly rounded f32 steps) against float64 exp:
  within one f32 ulp over the range, exact at 0, the clamps at -86 / 88.
- Known answers worked out by hand for inputs where the order decides the result: a team of
  lanes meeting in a pairwise tree (not in lane sequence), a lane's products entering its
  accumulator two at a time through the dot instruction's step (or_acc_step, pinned against the
  device in tests/test_oracle_arith.py; IEEE fused multiply-adds one by one give another value),
  and the sum of squares taken per 64-lane wave tree, then wave by wave.  A plausible slip
  (sequential lanes, one product at a time, the MLX order's 8 partials) gives a different value
  in each.
- Random rows: the device-order dot products and sums of squares against float64, within the
  f32 accumulation bound.
The DiT functions in this order are pinned by the same float64 restatements, closed forms and
invariants as in the MLX order (tests/test_oracle_dit.py runs every check in both orders)."""
import math

import numpy as np
import pytest

import oracle

BIG = 2.0 ** 24


def bits(vals):
    return oracle.to_bf16(np.asarray(vals, np.float32))


def test_exp_rep_vs_f64():
    rng = np.random.default_rng(5)
    xs = np.concatenate([np.linspace(-86.0, 88.0, 20001, dtype=np.float32),
                         rng.uniform(-20, 20, 20000).astype(np.float32),
                         rng.uniform(-1, 1, 5000).astype(np.float32)])
    worst = 0.0
    for x in xs:
        g = np.float32(oracle.exp_rep(float(x)))
        e = math.exp(float(x))
        ef = np.float32(e)
        ulp = float(np.spacing(ef))
        worst = max(worst, abs(float(g) - e) / ulp)
    assert worst <= 1.0, worst
    assert oracle.exp_rep(0.0) == 1.0
    assert oracle.exp_rep(-86.5) == 0.0 and oracle.exp_rep(-1e30) == 0.0
    assert math.isinf(oracle.exp_rep(88.5))
    assert math.isnan(oracle.exp_rep(float("nan")))


def test_dot_dev_lane_tree_known_answer():
    # K = 256, team 32: lane l holds chunk l (8 values).  Lane sums 2^24, 1, 1, 1, 0...:
    # pairwise tree -> (2^24 + 1 = 2^24, tie to even) + (1 + 1 = 2) = 2^24 + 2.
    # In lane sequence (or the MLX order, where all four sit in partial 0): 2^24.
    w = bits(np.ones(256))
    x = np.zeros(256, np.float32)
    x[0], x[8], x[16], x[24] = BIG, 1.0, 1.0, 1.0
    assert oracle.dot_dev(w, bits(x), 32) == BIG + 2
    # the same with 64-lane teams over K = 512
    w2 = bits(np.ones(512))
    x2 = np.zeros(512, np.float32)
    x2[0], x2[8], x2[16], x2[24] = BIG, 1.0, 1.0, 1.0
    assert oracle.dot_dev(w2, bits(x2), 64) == BIG + 2
    # lanes meet only after all their chunks: lane 0 takes chunks 0 and 32 (K = 512, team 32)
    x3 = np.zeros(512, np.float32)
    x3[0], x3[256], x3[8] = BIG, 1.0, 1.0  # lane 0: 2^24 + 1 = 2^24; lane 1: 1 -> 2^24 + 1 = 2^24
    assert oracle.dot_dev(w2, bits(x3), 32) == BIG


def test_dot_dev_element_order_known_answer():
    # one chunk [2^24, -0.75, 0, ...] with unit weights: both products enter in one dot2 step, whose
    # grid (1 here) truncates -0.75 to 0 -> 2^24.  One product at a time (fused multiply-adds):
    # 2^24 - 0.75 -> 2^24 - 1.
    w = bits(np.ones(8))
    assert oracle.dot_dev(w, bits([BIG, -0.75, 0, 0, 0, 0, 0, 0]), 32) == BIG
    # [1, 1, 2^24, 1, ...]: step 1 gives 2, step 2 adds 2^24 + 1 on the grid 1 -> 2^24 + 3 -> tie to
    # even 2^24 + 4 (pairs each rounded before the accumulator joins: 2^24 + 2)
    assert oracle.dot_dev(w, bits([1.0, 1.0, BIG, 1.0, 0, 0, 0, 0]), 32) == BIG + 4


def test_sumsq_dev_known_answer():
    # K = 1024: wave 0 holds chunks 0..63, wave 1 chunks 64..127.  Squares 2^24 (x = 2^12),
    # 1, 1, 1 in lanes 0..3 of wave 0 -> tree 2^24 + 2; wave 1 lane 0 -> 1; waves in order:
    # 2^24 + 3 -> 2^24 + 4 (tie to even).  All in sequence: 2^24.
    x = np.zeros(1024, np.float32)
    x[0], x[8], x[16], x[24], x[512] = 4096.0, 1.0, 1.0, 1.0, 1.0
    assert oracle.sumsq_dev(bits(x)) == BIG + 4


@pytest.mark.parametrize("K,team", [(64, 32), (256, 32), (896, 32), (1024, 32), (3584, 64), (4096, 64)])
def test_dot_dev_vs_f64(K, team):
    rng = np.random.default_rng(K + team)
    for _ in range(20):
        w = bits(rng.normal(0, 0.02, K))
        x = bits(rng.normal(0, 1, K))
        wf, xf = oracle.to_f32(w).astype(np.float64), oracle.to_f32(x).astype(np.float64)
        exact = float(wf @ xf)
        bound = (K / 8 + 4 * K / team) * 2 ** -24 * float(np.abs(wf) @ np.abs(xf))
        assert abs(oracle.dot_dev(w, x, team) - exact) <= bound


@pytest.mark.parametrize("K", [64, 896, 1024])
def test_sumsq_dev_vs_f64(K):
    rng = np.random.default_rng(K)
    for _ in range(20):
        x = bits(rng.normal(0, 1, K))
        xf = oracle.to_f32(x).astype(np.float64)
        exact = float(xf @ xf)
        assert abs(oracle.sumsq_dev(x) - exact) <= (8 + 7 + 2) * 2 ** -24 * exact


def test_order_switch_is_scoped():
    assert oracle.lib().or_get_dit_order() == oracle.DIT_ORDER_MLX
    with oracle.dit_order(oracle.DIT_ORDER_DEVICE):
        assert oracle.lib().or_get_dit_order() == oracle.DIT_ORDER_DEVICE
    assert oracle.lib().or_get_dit_order() == oracle.DIT_ORDER_MLX
