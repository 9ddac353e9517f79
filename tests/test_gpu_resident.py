"""Resident single steps (vvli_gpu_set_resident): forward_token calls handed
to a launch that stays on the stream, through pinned host memory.

Bar: bit-identical logits and argmax to separate single-step launches of the
same model (the same kernel and the same fixed summation orders), and the
oracle's argmax; covered: every return form, positions out of order, an idle
gap longer than the linger time (the launch has left: the next call
launches again), other entry points in between (each ends the launch first),
the last cache position and ContextFull, the device error path, the MoE step.
"""
import time

import numpy as np
import pytest

from vvli_amd import config as C
from vvli_amd import runtime as R
from vvli_amd._lib import VvliError

from test_gpu_forward import CASES, cfg_small, make_blob, rel_err
from test_gpu_moe import CASES as MOE_CASES
from test_gpu_moe import moe_blob

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _call(gpu, form, tok, pos):
    """(logits or None, argmax) of one call in the given return form."""
    if form == 0:
        return gpu.forward_token(tok, pos).copy(), gpu.last_argmax
    if form == 1:
        v = gpu.forward_token_view(tok, pos)
        return np.array(v), gpu.last_argmax
    return None, gpu.forward_token_argmax(tok, pos)


# Every resident kernel instance: head_dim 64 and 128 (exact), 32 and 96
# (the general instances); the MoE instances below.
RES_CASES = dict(CASES, hd32_g4=(cfg_small(num_attention_heads=8, num_key_value_heads=2), C.WEIGHT_BF16, "synth", 0))


@pytest.mark.parametrize("name", ["qwen_small", "llama_small", "hd128_g7", "hd32_g4", "hd96_g4"])
def test_resident_steps_equal_separate_launches(name, oracle_mod, host_threads):
    cfg, kind, how, _ = RES_CASES[name]
    blob = make_blob(cfg, kind, how)
    max_seq = 96
    rng = np.random.default_rng(11)
    # (token, pos, form): consecutive positions, then positions 5 and 6 again
    # with other tokens (the cache rows are overwritten), then onwards.
    plan = [(int(t), p, p % 3) for p, t in enumerate(rng.integers(0, cfg.vocab_size, size=24))]
    plan += [(int(rng.integers(0, cfg.vocab_size)), 5, 0), (int(rng.integers(0, cfg.vocab_size)), 6, 1)]
    plan += [(int(t), 7 + i, (i + 2) % 3) for i, t in enumerate(rng.integers(0, cfg.vocab_size, size=12))]
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    print(f"case={name} resident vs separate launches, {len(plan)} calls", flush=True)
    # Separate launches first: a resident launch idling on another stream
    # would hold every CU until its linger time runs out.
    refs = []
    with R.Runner(cfg, blob, max_seq) as ref:
        ref.set_decode_path("persistent")
        for i, (tok, pos, form) in enumerate(plan):
            logits, am = _call(ref, 0, tok, pos)
            refs.append((logits, am, ref.kv_read(0, 3) if i == 10 else None))
            assert am == oracle_mod.argmax(orc.forward_token(tok, pos)), f"call {i} pos {pos}: oracle argmax"
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path("persistent")
        gpu.set_resident(2000)
        for i, (tok, pos, form) in enumerate(plan):
            r_logits, r_am, r_kv = refs[i]
            g_logits, g_am = _call(gpu, form, tok, pos)
            assert g_am == r_am, f"call {i} pos {pos} form {form}: argmax"
            if g_logits is not None:
                assert np.array_equal(g_logits, r_logits), f"call {i} pos {pos} form {form}: logits differ"
            if r_kv is not None:  # another entry point in between: it ends the resident launch first
                k, v = gpu.kv_read(0, 3)
                assert np.array_equal(k, r_kv[0]) and np.array_equal(v, r_kv[1])
            if i in (20, 30):  # idle past the linger time: the launch leaves, the next call launches again
                time.sleep(0.05)


def test_resident_last_position_and_context_full(oracle_mod, host_threads):
    cfg, kind, how, _ = CASES["qwen_small"]
    max_seq = 40
    blob = make_blob(cfg, kind, how)
    orc = oracle_mod.OracleRunner(cfg, blob, max_seq, threads=host_threads)
    toks = np.random.default_rng(8).integers(0, cfg.vocab_size, size=max_seq)
    with R.Runner(cfg, blob, max_seq) as gpu:
        gpu.set_decode_path("persistent")
        gpu.set_resident(20000)
        for pos in range(max_seq):
            ref = orc.forward_token(int(toks[pos]), pos)
            got, am = _call(gpu, pos % 3, int(toks[pos]), pos)
            assert am == oracle_mod.argmax(ref), f"pos {pos}"
            if got is not None:
                assert rel_err(got, ref) <= TOL, f"pos {pos}"
        with pytest.raises(VvliError) as e:
            gpu.forward_token(int(toks[0]), max_seq)
        assert e.value.rc == 4
        with pytest.raises(VvliError):
            gpu.set_resident(100001)


def test_resident_error_is_reported(oracle_mod, host_threads):
    """The error path with resident steps: the test hook ends the resident
    launch and raises the device flag for the next launch, which leaves at
    once; the call reports VVLI_HIP_ERROR and the next calls run."""
    cfg, kind, how, _ = CASES["qwen_small"]
    blob = make_blob(cfg, kind, how)
    lib = R._lib.lib()
    toks = [5, 77, 300, 12, 9]
    orc = oracle_mod.OracleRunner(cfg, blob, 64, threads=host_threads)
    refs = [orc.forward_token(t, p) for p, t in enumerate(toks)]
    with R.Runner(cfg, blob, 64) as gpu:
        gpu.set_decode_path("persistent")
        gpu.set_resident(20000)
        gpu.forward_token(toks[0], 0)
        gpu.forward_token_argmax(toks[1], 1)
        R._lib.check(lib.vvli_gpu_test_inject_step_error(gpu._h, 1))
        with pytest.raises(VvliError) as e:
            gpu.forward_token_view(toks[2], 2)
        assert e.value.rc == 8 and "injected" in str(e.value)
        for pos in range(2, len(toks)):
            got, am = _call(gpu, pos % 3, toks[pos], pos)
            assert am == oracle_mod.argmax(refs[pos])
            if got is not None:
                assert rel_err(got, refs[pos]) <= TOL


@pytest.mark.parametrize("name,n", [("olmoe_small", 20), ("olmoe_1b_7b_2layers", 6)])
def test_resident_moe_steps_equal_separate_launches(name, n, oracle_mod):
    """MoE instances: head_dim 64 (the small case) and 128 (OLMoE-1B-7B layers)."""
    cfg, _ = MOE_CASES[name]
    blob = moe_blob(oracle_mod, cfg)
    toks = np.random.default_rng(4).integers(0, cfg.vocab_size, size=n)
    with R.MoeRunner(cfg, blob, 64) as ref:
        ref.set_decode_path("persistent")
        refs = [_call(ref, 0, int(tok), pos) for pos, tok in enumerate(toks)]
    with R.MoeRunner(cfg, blob, 64) as gpu:
        gpu.set_decode_path("persistent")
        gpu.set_resident(20000)
        for pos, tok in enumerate(toks):
            r_logits, r_am = refs[pos]
            g_logits, g_am = _call(gpu, pos % 3, int(tok), pos)
            assert g_am == r_am, f"pos {pos}: argmax"
            if g_logits is not None:
                assert np.array_equal(g_logits, r_logits), f"pos {pos}: logits differ"
