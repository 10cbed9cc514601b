"""The CFG decoding loop (ovh_lm_generate, tts.cpp:165-364): the restated host
logic is pinned here on the CPU; tests/test_gpu_lm.py runs the device loop
against it."""
import math
from fractions import Fraction

import numpy as np

import oracle


def test_mt19937_known_answer():
    """C++ [rand.predef]: the 10000th output of a default-constructed mt19937
    (seed 5489) is 4123659995."""
    assert int(oracle.mt19937_u32(5489, 10000)[-1]) == 4123659995


def test_uniform_float01_closed_form():
    x = np.array([0, 1, 2 ** 31, 2 ** 32 - 129, 2 ** 32 - 1], np.uint32)
    u = oracle.uniform_float01(x)
    assert u[0] == 0.0 and u[2] == 0.5
    assert np.all(u < 1.0) and u[-1] == np.nextafter(np.float32(1), np.float32(0))
    assert u.dtype == np.float32


def test_schedule():
    for steps, shift, total in [(32, 0.1, 8 * 260), (8, 0.1, 96), (5, 1.0, 10), (32, 0.1, 8)]:
        s = oracle.cfg_schedule(steps, shift, total)
        assert len(s) == steps and sum(s) == total and min(s) >= 0
    # t_shift = 1 is the identity grid: shares of ceil(total/steps), give or take
    # the one that double rounding of i/steps adds before the ceil
    s = oracle.cfg_schedule(5, 1.0, 10)
    assert all(abs(x - 2) <= 1 for x in s)
    # t_shift < 1 makes the grid convex: few positions first, more every step
    s = oracle.cfg_schedule(32, 0.1, 2080)
    assert all(a <= b for a, b in zip(s[:-2], s[1:-1])) and s[0] < s[-2]


def test_run_sampling_logic_with_a_stub_model():
    """With a stub step whose scores are fixed, the loop unmasks exactly the
    scheduled number of positions per step and writes each position once."""
    C_, V, S, T = 2, 9, 7, 4
    ids = np.full((C_, S), V - 1, np.int64)
    ids[:, :S - T] = 3
    am = np.zeros(S, np.uint8)
    am[S - T:] = 1
    calls = []

    def step(ids_b2, amask, attn, pos):
        calls.append(ids_b2.copy())
        assert attn[0].all() and attn[1, :T, :T].all() and attn[1, T:, T:].trace() == S - T
        pred = np.arange(C_ * T, dtype=np.int32).reshape(C_, T) % (V - 1)
        return pred, np.zeros((C_, T), np.float32)

    out = oracle.run_sampling(step, ids, am, T, C_, V, num_steps=4, t_shift=1.0)
    assert np.array_equal(out, (np.arange(C_ * T) % (V - 1)).reshape(C_, T))
    sched = oracle.cfg_schedule(4, 1.0, C_ * T)
    done = [(c[0][:, S - T:] != V - 1).sum() for c in calls]
    assert done == list(np.cumsum([0] + sched[:-1]))
    assert np.array_equal(calls[-1][1][:, :T], calls[-1][0][:, S - T:])


# tts.cpp:231-249 at the reference's defaults (32 steps, t_shift 0.1f, 8 codebooks x
# 260 frames).  By hand, step 0: ts_1 = 0.1 * (1/32) / (1 - 0.9/32) = 1/311, and
# ceil(2080/311) = ceil(6.688) = 7.
DEFAULT_SCHEDULE = [7, 8, 8, 8, 9, 10, 10, 11, 12, 13, 14, 15, 16, 17, 19, 21, 23, 26, 29, 32,
                    37, 42, 49, 57, 68, 82, 101, 128, 166, 226, 325, 491]


def _exact_schedule(steps, t_shift, total):
    """The schedule in exact rational arithmetic (t_shift as the float32 value the
    option holds): ts_i = a t / (1 + (a - 1) t), t = i / steps; per step
    ceil(total (ts_{s+1} - ts_s)) capped by what remains, the last step the rest."""
    a = Fraction(float(np.float32(t_shift)))
    ts = [a * Fraction(i, steps) / (1 + (a - 1) * Fraction(i, steps)) for i in range(steps + 1)]
    out, rem = [], total
    for s in range(steps):
        num = rem if s == steps - 1 else min(math.ceil(total * (ts[s + 1] - ts[s])), rem)
        out.append(num)
        rem -= num
    return out


def test_schedule_known_answer():
    """The restated schedule (double arithmetic, as tts.cpp) equals the known
    answer at the defaults, which the exact-rational closed form reproduces; a
    floor in place of the ceil, or i/steps in place of the shifted grid, would
    not (they change the per-step counts even where the sums agree)."""
    assert sum(DEFAULT_SCHEDULE) == 2080
    assert _exact_schedule(32, 0.1, 2080) == DEFAULT_SCHEDULE
    assert oracle.cfg_schedule(32, 0.1, 2080) == DEFAULT_SCHEDULE
    for steps, shift, total in [(8, 0.1, 96), (16, 0.5, 1000), (32, 0.1, 8 * 75), (4, 2.0, 33)]:
        assert oracle.cfg_schedule(steps, shift, total) == _exact_schedule(steps, shift, total)
