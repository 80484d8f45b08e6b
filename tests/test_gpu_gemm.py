"""GPU parity of the prefill projection GEMM (friday_gemm_q8) and the activation
quantiser (friday_quantize_q8_rows) against the CPU oracle.

Mirrors tests/kernels/test_prefill_gemm.cu: every weight kind at its three shapes
(T, K, N) = (1, 512, 64), (37, 1024, 200), (130, 768, 96) with bias + in-place residual,
random blocks with fp16 scales in [1e-3, 1e-2], x and res N(0,1), bias 0.1 N(0,1); the bar is
that test's (rel-L2 < 1e-3, max |diff| < 1e-2 of the RMS). The quantiser is bit-exact.
Adds a 32B-model projection shape on sampled rows and ldy > N with untouched padding.
"""
import numpy as np
import pytest

from fa_helpers import KQ_KINDS, assert_gemm_close, kq_random_weights

pytestmark = pytest.mark.gpu

SHAPES = [(1, 512, 64, False), (37, 1024, 200, False), (130, 768, 96, True)]


def run_gemm(fa, kind, W, x, T, K, N, bias=None, res=None, ldy=None, y_init=None):
    ldy = N if ldy is None else ldy
    dW = fa.DeviceBuffer.from_array(W)
    dx = fa.DeviceBuffer.from_array(x)
    dq = fa.DeviceBuffer(T * K)
    dd = fa.DeviceBuffer(T * (K // 32) * 4)
    fa.quantizeQ8Rows(dx, T, K, dq, dd)
    Y0 = np.zeros((T, ldy), np.uint16) if y_init is None else y_init
    dY = fa.DeviceBuffer.from_array(np.ascontiguousarray(Y0))
    db = fa.DeviceBuffer.from_array(bias) if bias is not None else None
    # residual in place, as the engine uses it: res and Y are the same buffer
    fa.gemmQ8(kind, dW, dq, dd, T, K, N, dY, ldy, bias=db, res=dY if res else None)
    fa.Hip.sync()
    return (dY.download((T, ldy), np.uint16), dq.download((T, K), np.int8),
            dd.download((T, K // 32), np.float32))


@pytest.mark.parametrize("T,K,N,epi", SHAPES)
@pytest.mark.parametrize("kind", sorted(KQ_KINDS))
def test_reference_gemm_cases(gpu, oracle, kind, T, K, N, epi):
    fa = gpu
    rng = np.random.default_rng(20261110 + 10 * kind + T)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    res = rng.standard_normal((T, N), dtype=np.float32).astype(np.float16).view(np.uint16)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32) if epi else None
    Y, xq, xd = run_gemm(fa, kind, W, x, T, K, N, bias=bias, res=epi, y_init=res if epi else None)
    oq, od = oracle.quantize_q8_rows(x)
    assert np.array_equal(xq, oq) and np.array_equal(xd.view(np.uint32), od.view(np.uint32))
    ref, _ = oracle.gemm_q8(kind, W, oq, od, T, K, N, bias=bias, res=res if epi else None)
    got = Y.view(np.float16).astype(np.float32)
    assert_gemm_close(got, ref.view(np.float16).astype(np.float32), f"{KQ_KINDS[kind][0]} T={T} K={K} N={N}")


def test_quantize_rows_edge_values(gpu, oracle):
    fa = gpu
    rng = np.random.default_rng(3)
    rows, K = 9, 1024
    x = (rng.standard_normal((rows, K), dtype=np.float32) * 5).astype(np.float16)
    x[0, :32] = 0                         # zero block: d = 0, q = 0
    x[1, 40] = np.float16(65504.0)        # fp16 max dominates its block
    x[2, 64:96] = np.float16(6e-8)        # subnormal block
    x[3, 100] = np.float16(-np.inf)       # amax = inf: d = inf, inv = 0
    dx = fa.DeviceBuffer.from_array(x.view(np.uint16))
    dq, dd = fa.DeviceBuffer(rows * K), fa.DeviceBuffer(rows * K // 32 * 4)
    fa.quantizeQ8Rows(dx, rows, K, dq, dd)
    fa.Hip.sync()
    oq, od = oracle.quantize_q8_rows(x.view(np.uint16))
    assert np.array_equal(dq.download((rows, K), np.int8), oq)
    assert np.array_equal(dd.download((rows, K // 32), np.float32).view(np.uint32), od.view(np.uint32))


def test_ldy_padding_untouched(gpu, oracle):
    fa = gpu
    kind, T, K, N, ldy = 3, 20, 512, 70, 96
    rng = np.random.default_rng(11)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    canary = np.full((T, ldy), 0x7BCD, np.uint16)
    Y, xq, xd = run_gemm(fa, kind, W, x, T, K, N, ldy=ldy, y_init=canary)
    assert (Y[:, N:] == 0x7BCD).all()
    ref, _ = oracle.gemm_q8(kind, W, xq, xd, T, K, N)
    assert_gemm_close(Y[:, :N].view(np.float16).astype(np.float32), ref.view(np.float16).astype(np.float32), "ldy")


@pytest.mark.parametrize("kind,K,N", [(1, 5120, 27648), (2, 27648, 5120), (3, 4096, 14336), (5, 14336, 4096)])
def test_model_projection_shapes(gpu, oracle, kind, K, N):
    """The reference's GEMM bench shapes (test_prefill_gemm.cu:40-42), T = 512; the oracle
    checks 48 sampled weight rows (every token), the rest only for finiteness."""
    fa = gpu
    T = 512
    rng = np.random.default_rng(kind + K)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    Y, xq, xd = run_gemm(fa, kind, W, x, T, K, N)
    got = Y.view(np.float16).astype(np.float32)
    assert np.isfinite(got).all()
    rows = np.unique(np.concatenate([[0, 1, 127, 128, N - 1], rng.choice(N, 43, replace=False)]))
    ref, _ = oracle.gemm_q8(kind, np.ascontiguousarray(W[rows]), xq, xd, T, K, len(rows))
    assert_gemm_close(got[:, rows], ref.view(np.float16).astype(np.float32), f"{KQ_KINDS[kind][0]} K={K} N={N}")


# ---- decode GEMV (friday_gemv_q8): test_kquant_kernels.cu shapes (K = 1024, N = 64) per kind,
# the O-projection of the decode step (transformer.cpp:1057-1059) at Qwen2.5-32B shapes with the
# residual in place, and the two-matrix launch (W2 -> y2) with a bias.

def run_gemv(fa, kind, W, x, K, N, W2=None, bias=None, res=None):
    dW = fa.DeviceBuffer.from_array(W)
    dW2 = fa.DeviceBuffer.from_array(W2) if W2 is not None else None
    dx = fa.DeviceBuffer.from_array(x)
    dq, dd = fa.DeviceBuffer(K), fa.DeviceBuffer(K // 32 * 4)
    fa.quantizeQ8Rows(dx, 1, K, dq, dd)
    dy = fa.DeviceBuffer.from_array(res if res is not None else np.zeros(N, np.uint16))
    dy2 = fa.DeviceBuffer.from_array(np.zeros(N, np.uint16)) if W2 is not None else None
    db = fa.DeviceBuffer.from_array(bias) if bias is not None else None
    fa.gemvQ8(kind, dW, dq, dd, K, N, dy, W2=dW2, y2=dy2, bias=db, res=dy if res is not None else None)
    fa.Hip.sync()
    y = dy.download(N, np.uint16)
    y2 = dy2.download(N, np.uint16) if W2 is not None else None
    return y, y2, dq.download((1, K), np.int8), dd.download((1, K // 32), np.float32)


@pytest.mark.parametrize("kind", sorted(KQ_KINDS))
def test_gemv_reference_kernel_shapes(gpu, oracle, kind):
    fa = gpu
    K, N = 1024, 64
    rng = np.random.default_rng(20261107 + kind)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((1, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    y, _, xq, xd = run_gemv(fa, kind, W, x, K, N)
    ref, _ = oracle.gemm_q8(kind, W, xq, xd, 1, K, N)
    assert_gemm_close(y.view(np.float16).astype(np.float32), ref.view(np.float16).astype(np.float32),
                      f"gemv {KQ_KINDS[kind][0]}")


@pytest.mark.parametrize("kind", [3, 5, 6])
def test_gemv_o_projection_residual(gpu, oracle, kind):
    fa = gpu
    K = N = 5120
    rng = np.random.default_rng(kind + 77)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((1, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    res = rng.standard_normal(N, dtype=np.float32).astype(np.float16).view(np.uint16)
    y, _, xq, xd = run_gemv(fa, kind, W, x, K, N, res=res)
    ref, _ = oracle.gemm_q8(kind, W, xq, xd, 1, K, N, res=res[None])
    assert_gemm_close(y.view(np.float16).astype(np.float32), ref[0].view(np.float16).astype(np.float32), "o_proj")


def test_gemv_two_matrices_bias(gpu, oracle):
    fa = gpu
    kind, K, N = 1, 2048, 300
    rng = np.random.default_rng(9)
    W, W2 = kq_random_weights(rng, kind, N, K), kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((1, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    y, y2, xq, xd = run_gemv(fa, kind, W, x, K, N, W2=W2, bias=bias)
    r1, _ = oracle.gemm_q8(kind, W, xq, xd, 1, K, N, bias=bias)
    r2, _ = oracle.gemm_q8(kind, W2, xq, xd, 1, K, N, bias=bias)
    f = lambda a: a.view(np.float16).astype(np.float32)  # noqa: E731
    assert_gemm_close(f(y), f(r1[0]), "y")
    assert_gemm_close(f(y2), f(r2[0]), "y2")


# ---- K split (shapes whose 128 x 128 tiles do not fill the GPU): fp32 partials in the
# library's per-stream workspace, summed in split order by the last workgroup of a tile.

SPLIT_SHAPES = [(256, 4096, 512, 3), (200, 2048, 384, 5), (512, 3072, 256, 6), (160, 4096, 300, 1)]


@pytest.mark.parametrize("T,K,N,kind", SPLIT_SHAPES)
def test_split_k_all_rows(gpu, oracle, T, K, N, kind):
    """Every output against the oracle, with bias and the residual in place."""
    fa = gpu
    rng = np.random.default_rng(T + K + N)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    res = rng.standard_normal((T, N), dtype=np.float32).astype(np.float16).view(np.uint16)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    Y, xq, xd = run_gemm(fa, kind, W, x, T, K, N, bias=bias, res=True, y_init=res)
    ref, _ = oracle.gemm_q8(kind, W, xq, xd, T, K, N, bias=bias, res=res)
    assert_gemm_close(Y.view(np.float16).astype(np.float32), ref.view(np.float16).astype(np.float32),
                      f"split {KQ_KINDS[kind][0]} T={T} K={K} N={N}")


def test_split_k_repeatable(gpu):
    """The tile counters re-arm: repeated calls, with a call of another split shape on the
    same stream in between, give identical bits."""
    fa = gpu
    rng = np.random.default_rng(5)
    kind, T, K, N = 3, 256, 4096, 512
    W = fa.DeviceBuffer.from_array(kq_random_weights(rng, kind, N, K))
    W2 = fa.DeviceBuffer.from_array(kq_random_weights(rng, kind, 256, 8192))
    dq, dd = fa.DeviceBuffer(T * 8192), fa.DeviceBuffer(T * 8192 // 32 * 4)
    x = rng.standard_normal((T, 8192), dtype=np.float32).astype(np.float16).view(np.uint16)
    fa.quantizeQ8Rows(fa.DeviceBuffer.from_array(x), T, 8192, dq, dd)
    dY, dY2 = fa.DeviceBuffer(T * N * 2), fa.DeviceBuffer(T * 256 * 2)
    outs = []
    for i in range(3):
        fa.gemmQ8(kind, W, dq, dd, T, K, N, dY, N)  # rows of xq read with stride K
        if i == 1:
            fa.gemmQ8(kind, W2, dq, dd, T, 8192, 256, dY2, 256)
        fa.Hip.sync()
        outs.append(dY.download((T, N), np.uint16))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_split_k_graph_replay(gpu, oracle):
    """gemmQ8Reserve before capture: the captured split GEMM replays bit-identically to the
    eager call; a stream with no workspace captures the unsplit GEMM, which also matches
    the oracle."""
    fa = gpu
    rng = np.random.default_rng(6)
    kind, T, K, N = 5, 256, 4096, 512
    Wh = kq_random_weights(rng, kind, N, K)
    W = fa.DeviceBuffer.from_array(Wh)
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    dq, dd = fa.DeviceBuffer(T * K), fa.DeviceBuffer(T * K // 32 * 4)
    fa.quantizeQ8Rows(fa.DeviceBuffer.from_array(x), T, K, dq, dd)
    fa.Hip.sync()
    eager = fa.DeviceBuffer(T * N * 2)
    fa.gemmQ8(kind, W, dq, dd, T, K, N, eager, N)
    fa.Hip.sync()
    ref_bits = eager.download((T, N), np.uint16)
    xq, xd = dq.download((T, K), np.int8), dd.download((T, K // 32), np.float32)
    ref, _ = oracle.gemm_q8(kind, Wh, xq, xd, T, K, N)
    for reserve in (True, False):
        stream = fa.Stream()
        if reserve:
            fa.gemmQ8Reserve(T, K, N, stream.s)
            stream.synchronize()
        dY = fa.DeviceBuffer(T * N * 2)
        graph = fa.Graph(stream, lambda: fa.gemmQ8(kind, W, dq, dd, T, K, N, dY, N, stream=stream.s))
        for _ in range(3):
            dY.fill_bytes(0)
            graph.launch()
            stream.synchronize()
            got = dY.download((T, N), np.uint16)
            if reserve:
                assert np.array_equal(got, ref_bits), "captured split GEMM differs from eager"
            assert_gemm_close(got.view(np.float16).astype(np.float32), ref.view(np.float16).astype(np.float32),
                              f"graph reserve={reserve}")


def test_caller_workspace_graphs(gpu):
    """friday_gemm_q8_ws: two graphs, each with its own workspace, captured on one stream and
    replayed alternately on two other streams, give the library-workspace call's bits on
    every replay (split K, 512 x 14336 -> 4096 as the 8B ffn_down)."""
    fa = gpu
    rng = np.random.default_rng(7)
    kind, T, K, N = 5, 512, 14336, 4096
    W = fa.DeviceBuffer.from_array(kq_random_weights(rng, kind, N, K))
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    dq, dd = fa.DeviceBuffer(T * K), fa.DeviceBuffer(T * K // 32 * 4)
    fa.quantizeQ8Rows(fa.DeviceBuffer.from_array(x), T, K, dq, dd)
    ref = fa.DeviceBuffer(T * N * 2)
    fa.gemmQ8(kind, W, dq, dd, T, K, N, ref, N)
    fa.Hip.sync()
    ref_bits = ref.download((T, N), np.uint16)
    nbytes = fa.gemmQ8WorkspaceBytes(T, K, N)
    cap = fa.Stream()
    graphs, outs = [], []
    for _ in range(2):
        ws = fa.DeviceBuffer(nbytes)
        fa.decodeWorkspaceInit(ws)
        fa.Hip.sync()
        y = fa.DeviceBuffer(T * N * 2)
        graphs.append(fa.Graph(cap, lambda ws=ws, y=y: fa.gemmQ8Ws(kind, W, dq, dd, T, K, N, y, N, ws, stream=cap.s)))
        outs.append((y, ws))
    runs = [fa.Stream(), fa.Stream()]
    for rep in range(3):
        for i, g in enumerate(graphs):
            outs[i][0].fill_bytes(0)
            fa.Hip.lib().hipGraphLaunch(g.exec, runs[(i + rep) % 2].s)
        fa.Hip.sync()
        for i in range(2):
            assert np.array_equal(outs[i][0].download((T, N), np.uint16), ref_bits), f"graph {i} replay {rep}"


@pytest.mark.parametrize("T,K,N,kind", [(130, 768, 96, 4), (37, 1024, 200, 1), (300, 1024, 2100, 6)])
def test_prehoisted_activations_bit_identical(gpu, T, K, N, kind):
    """The eager call dequantises the activations once into the workspace (fp16) and stages
    them from there; a call captured on a stream with no workspace dequantises them in every
    workgroup. Same values, same accumulation order (shapes with too few stages to split
    K): the outputs agree bit for bit."""
    fa = gpu
    rng = np.random.default_rng(T * N)
    W = fa.DeviceBuffer.from_array(kq_random_weights(rng, kind, N, K))
    x = rng.standard_normal((T, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    dq, dd = fa.DeviceBuffer(T * K), fa.DeviceBuffer(T * K // 32 * 4)
    fa.quantizeQ8Rows(fa.DeviceBuffer.from_array(x), T, K, dq, dd)
    eager = fa.DeviceBuffer(T * N * 2)
    fa.gemmQ8(kind, W, dq, dd, T, K, N, eager, N)
    fa.Hip.sync()
    stream = fa.Stream()  # fresh stream: no workspace, and none is allocated under capture
    dY = fa.DeviceBuffer(T * N * 2)
    graph = fa.Graph(stream, lambda: fa.gemmQ8(kind, W, dq, dd, T, K, N, dY, N, stream=stream.s))
    graph.launch()
    stream.synchronize()
    assert np.array_equal(dY.download((T, N), np.uint16), eager.download((T, N), np.uint16))


@pytest.mark.parametrize("kind,N", [(5, 63), (5, 62), (2, 61), (6, 70), (3, 65)])
def test_gemv_row_group_tails(gpu, oracle, kind, N):
    """Row counts that leave a short last row group; with an odd N and a 2-byte aligned kind
    (Q3_K, Q6_K, Q8_0) the groups would not span whole words and the direct kernel runs."""
    fa = gpu
    K = 2048
    rng = np.random.default_rng(kind * 100 + N)
    W = kq_random_weights(rng, kind, N, K)
    x = rng.standard_normal((1, K), dtype=np.float32).astype(np.float16).view(np.uint16)
    y, _, xq, xd = run_gemv(fa, kind, W, x, K, N)
    ref, _ = oracle.gemm_q8(kind, W, xq, xd, 1, K, N)
    assert_gemm_close(y.view(np.float16).astype(np.float32), ref.view(np.float16).astype(np.float32),
                      f"gemv tail {KQ_KINDS[kind][0]} N={N}")
