"""vvli_gpu_linear_noalloc (the allocation-free variant of the C2 op) against
vvli_gpu_linear, through the C ABI.

Two calls in a row, the second with a smaller input (the static scratch keeps
the first call's planes; nothing in it needs clearing), the GEMV path
(M < 4), and a call past the scratch limit (rejected before any launch, the
output untouched). Bar: bit-equal to vvli_gpu_linear wherever that op is
deterministic (two of its runs agree bit for bit), else -- split-K GEMMs add
partial sums with atomics in a varying order -- within 1e-5 max relative
error; and within the C2 bar of 2e-3 of the oracle's linearInto on sampled
rows.
"""
import numpy as np
import pytest

from vvli_amd import runtime as R
from vvli_amd._lib import VvliError

pytestmark = pytest.mark.gpu

LIMIT = 16 << 20  # VVLI_LINEAR_NOALLOC_SCRATCH_BYTES


def bf16_bits(a: np.ndarray) -> np.ndarray:
    b = a.astype(np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def rel_err(got, ref) -> float:
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def run_case(M, N, K, has_bias, oracle_mod, seed):
    import torch

    rng = np.random.default_rng(seed)
    w = bf16_bits(rng.normal(0, 0.02, size=(N, K)))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    bias = bf16_bits(rng.normal(0, 0.02, size=N)) if has_bias else None
    dev = torch.device("cuda", 0)
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    db = torch.from_numpy(bias.view(np.int16)).to(dev) if has_bias else None
    bptr = None if db is None else db.data_ptr()
    outs = []
    for fn in (R.linear, R.linear, R.linear_noalloc):
        dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        fn(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K, bptr)
        torch.cuda.synchronize()
        outs.append(dy.cpu().numpy())
    a, a2, got = outs
    assert np.isfinite(got).all()
    if np.array_equal(a.view(np.uint32), a2.view(np.uint32)):
        assert np.array_equal(got.view(np.uint32), a.view(np.uint32)), f"M={M} N={N} K={K}: not bit-equal"
    else:
        e = rel_err(got, a)
        assert e <= 1e-5, f"M={M} N={N} K={K}: rel err {e:.2e} against vvli_gpu_linear"
    for m in sorted({0, M // 2, M - 1}):
        e = rel_err(got[m], oracle_mod.linear(w, x[m], bias))
        assert e <= 2e-3, f"M={M} N={N} K={K} row {m}: rel err {e:.2e} against the oracle"


def test_noalloc_linear_matches_linear(oracle_mod):
    # First call: the largest split that fits (4 * 512 * 8192 bytes = the whole scratch).
    assert 4 * 512 * 8192 == LIMIT
    print("noalloc call 1: M=512 N=2048 K=8192", flush=True)
    run_case(512, 2048, 8192, False, oracle_mod, 1)
    # Second call, smaller: stale planes of the first call remain beyond its
    # rows; the skinny kernel with K split across blocks (32 row tiles, 2
    # splits): its counters and partials in the same scratch.
    print("noalloc call 2: M=64 N=512 K=4096 bias", flush=True)
    run_case(64, 512, 4096, True, oracle_mod, 2)
    print("noalloc call 3: M=130 N=1000 K=896 bias (ragged tiles)", flush=True)
    run_case(130, 1000, 896, True, oracle_mod, 3)
    print("noalloc call 4: M=2 N=2048 K=2048 (GEMV path)", flush=True)
    run_case(2, 2048, 2048, False, oracle_mod, 4)


def test_noalloc_linear_rejects_oversize():
    import torch

    dev = torch.device("cuda", 0)
    M, N, K = 513, 64, 8192  # 4 * 513 * 8192 bytes > the scratch
    dw = torch.zeros((N, K), dtype=torch.int16, device=dev)
    dx = torch.zeros((M, K), dtype=torch.float32, device=dev)
    dy = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    print("noalloc oversize call", flush=True)
    with pytest.raises(VvliError) as e:
        R.linear_noalloc(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K)
    assert e.value.name == "InvalidConfig"
    torch.cuda.synchronize()
    assert bool((dy == 7.0).all())


@pytest.mark.parametrize("M,N,K,has_bias", [
    (16, 512, 8192, False),  # skinny MFMA with K split across blocks (32 row tiles): counters in the scratch
    (130, 1000, 896, True),  # the GEMM path: activation split planes in the scratch
])
def test_noalloc_linear_in_graph(M, N, K, has_bias, oracle_mod):
    """vvli_gpu_linear_noalloc captured into a HIP graph (torch.cuda.CUDAGraph
    over the entry point on the capture stream): after one eager call on the
    device (its one-time set-up: attributes and the scratch address), the
    capture records kernels only (neither path issues a memset), and every
    replay -- three, with other eager calls and synchronisations between them
    -- matches the eager result: bit-equal where the op is deterministic,
    else within 1e-5."""
    import torch

    rng = np.random.default_rng(M + N + K)
    w = bf16_bits(rng.normal(0, 0.02, size=(N, K)))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    bias = bf16_bits(rng.normal(0, 0.02, size=N)) if has_bias else None
    dev = torch.device("cuda", 0)
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    bptr = None if bias is None else torch.from_numpy(bias.view(np.int16)).to(dev)
    bp = None if bptr is None else bptr.data_ptr()
    stream = torch.cuda.Stream(device=dev)
    eager = []
    for _ in range(2):
        dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        R.linear_noalloc(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K, bp, stream=stream.cuda_stream)
        stream.synchronize()
        eager.append(dy.cpu().numpy())
    deterministic = np.array_equal(eager[0].view(np.uint32), eager[1].view(np.uint32))
    assert rel_err(eager[0][0], oracle_mod.linear(w, x[0], bias)) <= 2e-3
    yg = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    g = torch.cuda.CUDAGraph()
    print(f"noalloc graph capture M={M} N={N} K={K}", flush=True)
    with torch.cuda.graph(g, stream=stream):
        R.linear_noalloc(dw.data_ptr(), dx.data_ptr(), yg.data_ptr(), M, N, K, bp, stream=stream.cuda_stream)
    # Between replays: an eager call that uses the same static scratch (a
    # skinny K-split call: its counters and partials).
    other = torch.zeros((16, 512), dtype=torch.float32, device=dev)
    ow = torch.zeros((512, 2048), dtype=torch.int16, device=dev)
    ox = torch.ones((16, 2048), dtype=torch.float32, device=dev)
    for rep in range(3):
        yg.fill_(float("nan"))
        with torch.cuda.stream(stream):
            g.replay()
        stream.synchronize()
        got = yg.cpu().numpy()
        if deterministic:
            assert np.array_equal(got.view(np.uint32), eager[0].view(np.uint32)), f"replay {rep}: not bit-equal"
        else:
            e = rel_err(got, eager[0])
            assert e <= 1e-5, f"replay {rep}: rel err {e:.2e}"
        # eager work between replays on the same scratch
        R.linear_noalloc(ow.data_ptr(), ox.data_ptr(), other.data_ptr(), 16, 512, 2048)
        torch.cuda.synchronize()
        assert bool((other == 0).all())
    del g
