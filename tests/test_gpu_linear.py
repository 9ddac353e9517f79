"""GPU parity of the C2 op (vvli_gpu_linear: Y[m,n] = sum_k bf16 W[n,k] *
X[m,k] (+ bias[n]), f32 accumulation) against the oracle's linearInto
restatement (oracle/vvli_oracle.c, src/llm.zig:1228-1285), row by row.

Bar: per output row, max |gpu - ref| / max |ref| <= 2e-3 (f32 accumulation
on both sides; the order of the K sum differs)."""
import numpy as np
import pytest

from vvli_amd import runtime as R
from vvli_amd._lib import VvliError

pytestmark = pytest.mark.gpu

TOL = 2e-3

# (M, N, K, bias): decode shapes of the benchmark model at M = 1, small and
# ragged ones, and M > 1 (the reference runs M independent linearInto calls;
# from M = 4 the library runs one MFMA GEMM).
SHAPES = [
    (1, 2048, 2048, False),
    (1, 512, 2048, False),
    (3, 1000, 896, True),
    (8, 2048, 8192, False),
    (17, 333, 64, True),
    (64, 1024, 2048, False),
    # GEMM path (M >= 4): prefill-sized rows, ragged tiles, stacked-output widths.
    (4, 130, 24, True),
    (128, 3072, 2048, False),
    (130, 1000, 896, True),
    (512, 2048, 2048, True),
    (300, 8192, 128, False),
    (33, 257, 4864, True),
    # Skinny MFMA path (4 <= M <= 64): 32-row blocks with a ragged last block,
    # K not a multiple of the 32-wide step, M just past a 16-row tile.
    (5, 8200, 2056, True),
    (63, 100, 40, False),
    (16, 8192, 896, False),
]


def bf16_bits(a: np.ndarray) -> np.ndarray:
    b = a.astype(np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)  # RNE (src/llm.zig:799-803)


@pytest.mark.parametrize("M,N,K,has_bias", SHAPES)
def test_linear_matches_oracle(M, N, K, has_bias, oracle_mod):
    import torch

    rng = np.random.default_rng(M * 100003 + N * 7 + K)
    w = bf16_bits(rng.normal(0, 0.02, size=(N, K)))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    bias = bf16_bits(rng.normal(0, 0.02, size=N)) if has_bias else None
    dev = torch.device("cuda", 0)
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.zeros((M, N), dtype=torch.float32, device=dev)
    db = torch.from_numpy(bias.view(np.int16)).to(dev) if has_bias else None
    print(f"linear M={M} N={N} K={K} bias={has_bias}", flush=True)
    R.linear(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K, None if db is None else db.data_ptr())
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    for m in range(M):
        ref = oracle_mod.linear(w, x[m], bias)
        e = float(np.max(np.abs(y[m] - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
        assert e <= TOL, f"row {m}: rel err {e:.3e}"


def test_linear_rejects_bad_shapes():
    import torch

    dev = torch.device("cuda", 0)
    w = torch.zeros((16, 12), dtype=torch.int16, device=dev)
    x = torch.zeros((1, 12), dtype=torch.float32, device=dev)
    y = torch.zeros((1, 16), dtype=torch.float32, device=dev)
    with pytest.raises(VvliError):  # K must be a multiple of 8
        R.linear(w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 16, 12)
    with pytest.raises(VvliError):  # NULL pointer
        R.linear(0, x.data_ptr(), y.data_ptr(), 1, 16, 8)


def test_linear_two_streams_growing_scratch(oracle_mod):
    """Calls on two streams, interleaved, with M growing (the per-stream split
    scratch is reallocated stream-ordered) and shrinking: every result matches
    the oracle; a call queued behind a larger one on the same stream reuses
    its scratch."""
    import torch

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7)
    N, K = 384, 512
    w = bf16_bits(rng.normal(0, 0.02, size=(N, K)))
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    jobs = []
    for i, M in enumerate([4, 8, 64, 200, 16, 130]):
        x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
        dx = torch.from_numpy(x).to(dev)
        dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        s = streams[i % 2]
        R.linear(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K, stream=s.cuda_stream)
        jobs.append((x, dx, dy))
    torch.cuda.synchronize()
    for x, _, dy in jobs:
        y = dy.cpu().numpy()
        for m in range(x.shape[0]):
            ref = oracle_mod.linear(w, x[m], None)
            e = float(np.max(np.abs(y[m] - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
            assert e <= TOL, f"M={x.shape[0]} row {m}: rel err {e:.3e}"


_BENCH_W = {}


def _bench_weights(N, K):
    if (N, K) not in _BENCH_W:
        _BENCH_W.clear()
        rng = np.random.default_rng(N + K)
        w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        _BENCH_W[(N, K)] = bf16_bits(w)
    return _BENCH_W[(N, K)]


# The isolated op sweep on the Llama-3.2-1B projection shapes: q/o, k/v,
# gate/up, down and lm_head, each at every M of the sweep.
SWEEP_SHAPES = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192), (128256, 2048)]
SWEEP_M = [1, 4, 16, 128, 512]


@pytest.mark.parametrize("M", SWEEP_M)  # M varies fastest: each weight matrix is generated once
@pytest.mark.parametrize("N,K", SWEEP_SHAPES)
def test_linear_benchmark_shapes(N, K, M, oracle_mod):
    """Every (N, K) x M point of the op sweep the benchmark times: GEMV
    (M = 1), skinny MFMA (4, 16) and GEMM (128, 512) paths. Every row of x
    for M <= 16; for M = 128 / 512 the rows at the edges of the GEMM's
    16-row fragments and 128-row block tiles, the middle and the last, each
    compared with the oracle over all N outputs."""
    import torch

    w = _bench_weights(N, K)
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, K), dtype=np.float32)
    dev = torch.device("cuda", 0)
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    print(f"linear bench shape M={M} N={N} K={K}", flush=True)
    R.linear(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K)
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    assert np.isfinite(y).all()
    rows = range(M) if M <= 16 else sorted({0, 1, 15, 16, 63, 64, 127, M // 2, M - 1} & set(range(M)) |
                                          ({128, 129, 255, 256, 383, 384} & set(range(M))))
    for m in rows:
        ref = oracle_mod.linear(w, x[m], None)
        e = float(np.max(np.abs(y[m] - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
        assert e <= TOL, f"M={M} N={N} row {m}: rel err {e:.3e}"


@pytest.mark.parametrize("M,N,K,has_bias", [
    (1, 37, 40, True),      # rows of 5 units: one unit per lane, most lanes masked
    (2, 4099, 896, False),  # 112 units per row (two per lane, a ragged second), ragged last block
    (3, 130, 8192, True),   # three rows of x in one launch, 4 items per row
    (2, 1, 2048, True),     # a single output row
    (3, 512, 16384, False), # 3 x 64 KiB of x exceeds LDS: one launch per row
    (1, 300, 40960, False), # the largest K whose x fits LDS
    (4, 300, 2048, True),   # M = 4 where the skinny row tiles leave CUs idle: four rows of x in one launch
    (4, 1000, 10240, False),  # M = 4, the largest K whose four x rows fit LDS
    (4, 700, 10248, True),  # M = 4 past that: the skinny kernel
])
def test_linear_gemv_shapes(M, N, K, has_bias, oracle_mod):
    """The GEMV kernel (M <= 3, and M = 4 where the skinny kernel's row tiles
    leave CUs idle: one launch for up to four rows of x staged in LDS, whole-row wave tiles
    walked in items of 1-4 units per lane): ragged rows and tiles, bias, and
    the per-row fallback, against the oracle."""
    import torch

    rng = np.random.default_rng(M * 31 + N * 17 + K)
    w = bf16_bits(rng.normal(0, 0.02, size=(N, K)))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    bias = bf16_bits(rng.normal(0, 0.02, size=N)) if has_bias else None
    dev = torch.device("cuda", 0)
    dw = torch.from_numpy(w.view(np.int16)).to(dev)
    dx = torch.from_numpy(x).to(dev)
    dy = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    db = torch.from_numpy(bias.view(np.int16)).to(dev) if has_bias else None
    print(f"linear gemv M={M} N={N} K={K} bias={has_bias}", flush=True)
    R.linear(dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), M, N, K, None if db is None else db.data_ptr())
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    for m in range(M):
        ref = oracle_mod.linear(w, x[m], bias)
        e = float(np.max(np.abs(y[m] - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
        assert e <= TOL, f"M={M} N={N} K={K} row {m}: rel err {e:.3e}"


def test_linear_gemv_rejects_k_beyond_lds():
    """M <= 3 stages x in LDS: K beyond 40960 floats is an invalid shape for
    those M (checked before any launch)."""
    import torch

    dev = torch.device("cuda", 0)
    K = 40968
    w = torch.zeros((4, K), dtype=torch.int16, device=dev)
    x = torch.zeros((1, K), dtype=torch.float32, device=dev)
    y = torch.zeros((1, 4), dtype=torch.float32, device=dev)
    with pytest.raises(VvliError):
        R.linear(w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 4, K)
