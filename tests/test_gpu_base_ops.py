"""The plugin's f32 tensor-op slots against the reference CPU backend's
semantics (src/cpu_backend.cpp:185-266): elementwise add/sub/mul (and div)
are one IEEE fp32 operation per element, matmul sums every output in
ascending k with a separate multiply and add.  Both are bit-exact here:
numpy float32 elementwise ops, and a float32 loop over k for matmul.  The
reference's own known answer (test/test_core.cpp:95-117) is checked too.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def seq_matmul(a, b):
    """C = A . B in float32, k ascending, multiply then add per step."""
    M, K = a.shape
    N = b.shape[1]
    c = np.zeros((M, N), np.float32)
    for k in range(K):
        c = (c + np.outer(a[:, k], b[k, :]).astype(np.float32)).astype(np.float32)
    return c


def gpu_binary(ctx, op, a, b):
    A, B = ctx.upload(a), ctx.upload(b)
    O = ctx.alloc(max(4, a.nbytes))
    try:
        ctx.binary_f32(op, A, B, O, a.size)
        return O.download(np.float32, a.shape)
    finally:
        for t in (A, B, O):
            t.free()


def test_capabilities(ctx):
    from mlx_amd import abi
    caps = ctx.be.desc.capabilities
    assert caps & abi.CAP_TENSOR_OPS and caps & abi.CAP_MATMUL
    assert not caps & (1 << 5)  # never UNIFIED_MEMORY: a discrete GPU


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 65536 + 7])
def test_elementwise_bit_exact(ctx, n):
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b[b == 0] = 1.0
    with np.errstate(all="ignore"):
        want = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}
    for op, w in want.items():
        print(f"[case] op_{op}_f32 n={n}", flush=True)
        got = gpu_binary(ctx, op, a, b)
        assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), op


def test_elementwise_special_values(ctx):
    a = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, 3.0e38, 1.0], np.float32)
    b = np.array([0.0, 0.0, 0.0, -0.0, np.inf, np.inf, 1.0, 2.0, 3.0e38, 1e-45], np.float32)
    with np.errstate(all="ignore"):
        want = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}
    for op, w in want.items():
        got = gpu_binary(ctx, op, a, b)
        nan = np.isnan(w)
        assert np.array_equal(np.isnan(got), nan), op
        assert np.array_equal(got[~nan].view(np.uint32), w[~nan].view(np.uint32)), op


def test_matmul_reference_kat(ctx):
    """test/test_core.cpp:95-117: [[1,2],[3,4]] . [[5,6],[7,8]] = [[19,22],[43,50]]."""
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    A, B, C = ctx.upload(a), ctx.upload(b), ctx.alloc(16)
    ctx.matmul_f32(A, B, C, 2, 2, 2)
    got = C.download(np.float32, (2, 2))
    for t in (A, B, C):
        t.free()
    assert np.array_equal(got, np.array([[19, 22], [43, 50]], np.float32))


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 5, 7), (64, 64, 64), (65, 33, 129), (130, 257, 70), (7, 0, 5)])
def test_matmul_bit_exact(ctx, M, K, N):
    rng = np.random.default_rng(M * 1000 + K * 10 + N)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    print(f"[case] op_matmul_f32 M={M} K={K} N={N}", flush=True)
    A, B, C = ctx.upload(a if a.size else np.zeros(1, np.float32)), \
        ctx.upload(b if b.size else np.zeros(1, np.float32)), ctx.alloc(M * N * 4)
    ctx.matmul_f32(A, B, C, M, K, N)
    got = C.download(np.float32, (M, N))
    for t in (A, B, C):
        t.free()
    assert np.array_equal(got.view(np.uint32), seq_matmul(a, b).view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 70), (64, 32), (129, 65)])
def test_transpose_exact(ctx, rows, cols):
    a = np.random.default_rng(rows * cols).standard_normal((rows, cols)).astype(np.float32)
    A, O = ctx.upload(a), ctx.alloc(a.nbytes)
    ctx.transpose_f32(A, O, rows, cols)
    got = O.download(np.float32, (cols, rows))
    A.free()
    O.free()
    assert np.array_equal(got, a.T)


def test_size_checks(ctx):
    """Counts past a buffer's size are INVALID_ARGUMENT, not a fault."""
    from mlx_amd import abi, runtime
    A, B, O = ctx.alloc(64), ctx.alloc(64), ctx.alloc(64)
    for call in (lambda: ctx.binary_f32("add", A, B, O, 17),
                 lambda: ctx.matmul_f32(A, B, O, 4, 5, 4),
                 lambda: ctx.transpose_f32(A, O, 4, 5)):
        with pytest.raises(runtime.LuxError) as e:
            call()
        assert e.value.code == abi.ERR_INVALID_ARGUMENT
    ctx.binary_f32("add", A, B, O, 16)  # exactly the buffer
    ctx.sync()
    for t in (A, B, O):
        t.free()
