"""The oracle's sampler (oracle/vvli_oracle_sample.c) against the reference's
own sampler tests (src/generator.zig:491-512), closed forms, the published
SplitMix64 sequence and the published xoshiro256++ known-answer vector (Zig's
std, which holds DefaultPrng, is not in the reference tree)."""
import ctypes
import math

import numpy as np
import pytest

from vvli_amd import _lib
from vvli_amd import runtime as R


def opts(**kw):
    base = dict(temperature=0.8, top_p=0.95, top_k=40, repeat_penalty=1.10, repeat_last_n=64, seed=0)
    base.update(kw)
    return R.Sampling(**base)


def test_splitmix64_published_sequence(oracle_mod):
    s = ctypes.c_uint64(0)
    got = [oracle_mod.lib().orc_splitmix64_next(ctypes.byref(s)) for _ in range(4)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    # DefaultPrng.init: the state is four SplitMix64 outputs.
    assert [int(x) for x in oracle_mod.prng_seed(0)] == got


# xoshiro256++ from state {1, 2, 3, 4}: the first ten outputs of Blackman and Vigna's reference
# implementation (the known-answer vector Rust's rand_xoshiro also checks).
XOSHIRO256PP_1234 = [41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205,
                     9973669472204895162, 14011001112246962877, 12406186145184390807, 15849039046786891736,
                     10450023813501588000]


def test_xoshiro256pp_published_vector(oracle_mod):
    st = np.array([1, 2, 3, 4], dtype=np.uint64)
    got = [int(oracle_mod.lib().orc_prng_next(oracle_mod._p(st))) for _ in range(10)]
    assert got == XOSHIRO256PP_1234


def test_float_f32_on_the_published_stream(oracle_mod):
    """Random.float(f32): 23 mantissa bits from the output's low bits, exponent 126 - clz(output).
    The first five outputs have 38, 38, 12, 12 and 0 leading zeros: 0x2800001 -> 2^-39 * (1 + 2^-23),
    0x3800067 -> exponent 88 with mantissa 0x67, and the fifth (>= 2^63) lands in [0.5, 1)."""
    st = np.array([1, 2, 3, 4], dtype=np.uint64)
    bits = [int(np.float32(oracle_mod.lib().orc_prng_float(oracle_mod._p(st))).view(np.uint32)) for _ in range(5)]
    assert bits == [0x2C000001, 0x2C000067, 0x39000067, 0x394400B2, 0x3F4433CD]
    assert np.float32(np.uint32(0x2C000001).view(np.float32)) == np.float32(2.0**-39 * (1 + 2.0**-23))
    # Each draw consumed exactly one output: the state now yields the sixth.
    assert int(oracle_mod.lib().orc_prng_next(oracle_mod._p(st))) == XOSHIRO256PP_1234[5]


def test_library_seed_mapping_matches_oracle(oracle_mod):
    # Sampler.init maps seed 0 to 0x9e3779b97f4a7c15 (src/generator.zig:75).
    assert np.array_equal(R.prng_seed(0), oracle_mod.prng_seed(0x9E3779B97F4A7C15))
    assert np.array_equal(R.prng_seed(12345), oracle_mod.prng_seed(12345))


def test_prng_float_range_and_mean(oracle_mod):
    st = oracle_mod.prng_seed(7)
    u = np.array([oracle_mod.lib().orc_prng_float(oracle_mod._p(st)) for _ in range(20000)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(np.mean(u < 0.25) - 0.25) < 0.015


def test_reference_repeat_penalty_greedy(oracle_mod):
    # src/generator.zig:491-499: counts [1, 0, 0], penalty 2 moves the choice to 1.
    logits = np.array([10.0, 9.8, 1.0], np.float32)
    counts = np.array([1, 0, 0], np.uint16)
    assert oracle_mod.lib().orc_greedy_with_penalties(oracle_mod._p(logits), oracle_mod._p(counts), 3, 2.0) == 1
    st = oracle_mod.prng_seed(1)
    o = opts(temperature=0.0, repeat_penalty=2.0)
    assert oracle_mod.sampler_next(logits, [0], [], o, st) == 1  # token 0 in the window
    assert oracle_mod.sampler_next(logits, [2], [], o, st) == 0


def build_candidates(oracle_mod, logits, counts, o):
    lg = np.ascontiguousarray(logits, np.float32)
    c = np.ascontiguousarray(counts, np.uint16)
    ids = np.zeros(lg.size, np.uint32)
    sc = np.zeros(lg.size, np.float32)
    so = oracle_mod.orc_sampling(o)
    n = oracle_mod.lib().orc_build_candidates(oracle_mod._p(ids), oracle_mod._p(sc), oracle_mod._p(lg),
                                              oracle_mod._p(c), lg.size, ctypes.byref(so))
    return ids[:n], sc[:n]


def test_reference_top_k_builder(oracle_mod):
    # src/generator.zig:501-512: top_k 2 over [1, 4, 2, 3] keeps ids 1 and 3.
    ids, sc = build_candidates(oracle_mod, [1.0, 4.0, 2.0, 3.0], [0, 0, 0, 0], opts(top_k=2, top_p=1.0))
    assert list(ids) == [1, 3] and list(sc) == [4.0, 3.0]


def test_candidates_ties_nonfinite_and_penalty(oracle_mod):
    lg = [1.0, np.nan, 5.0, np.inf, 5.0, -np.inf, 3.0, 5.0]
    ids, sc = build_candidates(oracle_mod, lg, [0] * 8, opts(top_k=3))
    assert list(ids) == [2, 4, 7]  # equal logits: lower id first; NaN / inf dropped
    ids, _ = build_candidates(oracle_mod, lg, [0] * 8, opts(top_k=0))
    assert list(ids) == [2, 4, 7, 6, 0]
    # Penalty: positive logits divided, negative multiplied (adjustedLogit, :391-394).
    ids, sc = build_candidates(oracle_mod, [2.0, -2.0, 1.5], [1, 1, 0], opts(top_k=0, repeat_penalty=2.0))
    assert list(ids) == [2, 0, 1] and list(sc) == [1.5, 1.0, -4.0]


def test_probabilities_and_pick_closed_form(oracle_mod):
    L = oracle_mod.lib()
    scores = np.array([2.0, 1.0, 0.0], np.float32)
    probs = np.zeros(3, np.float32)
    so = oracle_mod.orc_sampling(opts(temperature=1.0, top_p=0.7))
    k = L.orc_prepare_probabilities(oracle_mod._p(probs), oracle_mod._p(scores), 3, ctypes.byref(so))
    np.testing.assert_allclose(probs, [1.0, math.exp(-1), math.exp(-2)], rtol=1e-6)
    assert k == 2  # 1/1.503 < 0.7 <= 1.368/1.503
    so = oracle_mod.orc_sampling(opts(temperature=1.0, top_p=1.0))
    assert L.orc_prepare_probabilities(oracle_mod._p(probs), oracle_mod._p(scores), 3, ctypes.byref(so)) == 3
    ids = np.array([10, 20, 30], np.uint32)
    pick = lambda u, n: L.orc_sample_candidate(oracle_mod._p(ids), oracle_mod._p(probs), n, u)
    total2 = 1 + math.exp(-1)
    assert pick(0.5, 2) == 10  # target 0.684 <= 1
    assert pick(0.9, 2) == 20  # target 1.231 > 1
    assert pick(1.0, 2) == 20  # u clamped to 0.99999994
    assert pick(1.0 / total2 - 1e-6, 2) == 10
    # Temperature below 1e-6 is raised to 1e-6 (prepareProbabilities, :430).
    so = oracle_mod.orc_sampling(opts(temperature=1e-9, top_p=1.0))
    L.orc_prepare_probabilities(oracle_mod._p(probs), oracle_mod._p(scores), 3, ctypes.byref(so))
    assert list(probs) == [1.0, 0.0, 0.0]


def test_invalid_options(oracle_mod):
    st = oracle_mod.prng_seed(1)
    lg = np.zeros(4, np.float32)
    for bad in (dict(temperature=-1.0), dict(top_p=0.0), dict(top_p=1.5), dict(repeat_penalty=0.5),
                dict(temperature=float("nan"))):
        with pytest.raises(oracle_mod.OracleError) as e:
            oracle_mod.sampler_next(lg, [0], [], opts(**bad), st)
        assert e.value.rc == 15
