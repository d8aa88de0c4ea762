"""The int8 lm_head GEMV (gemv_i8w, src/kernels/gemv_i8w.cl:55-106) on the GPU against the
oracle's restatement (one fp32 chain over k, then the column's scale) and fp64.

Bar: the logits tolerance, rel 2e-3 of each value plus 2e-3 of the row's largest; against
fp64 the fp32 summation bound of the products (exact in fp32) for the matrix core's order."""
import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu


def untile(qt, K, N):
    """mi_i8w_index's layout [N/16][K/64][q 4][n 16][half 2][e 8] -> row-major [N][K]
    (n = 16 t + n16, k = 64 c + 32 half + 8 q + e)."""
    a = qt.reshape(N // 16, K // 64, 4, 16, 2, 8)
    return np.ascontiguousarray(a.transpose(0, 3, 1, 4, 2, 5)).reshape(N, K)


def test_layout_inverse_matches_the_index():
    K, N = 128, 32
    qt = np.arange(K * N, dtype=np.int64)
    rm = untile(qt, K, N)
    L = mi.lib()
    for n in (0, 5, 17, 31):
        for k in (0, 7, 8, 33, 63, 64, 127):
            assert rm[n, k] == L.mi_i8w_index(K, k, n)


@pytest.mark.parametrize("M,K,N", [(1, 512, 1024), (3, 512, 1024), (8, 1024, 256), (1, 5120, 151936)])
def test_gemv_i8w_vs_oracle_and_fp64(M, K, N):
    rng = np.random.default_rng(M + K)
    qt = rng.integers(-127, 128, K * N, dtype=np.int64).astype(np.int8)
    s = rng.uniform(2e-4, 2e-3, N).astype(np.float32)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    print(f"gemv_i8w M={M} K={K} N={N}", flush=True)
    dq, ds, dx = dev(qt), dev(s), dev(x)
    out = empty((M, N), np.float32)
    mi.call("mi_gemv_i8w", ptr(dq), ptr(ds), ptr(dx), ptr(out), M, K, N, stream())
    sync()
    got = host(out, np.float32)
    again = empty((M, N), np.float32)
    mi.call("mi_gemv_i8w", ptr(dq), ptr(ds), ptr(dx), ptr(again), M, K, N, stream())
    sync()
    assert np.array_equal(host(again, np.uint32), host(out, np.uint32))  # replays bitwise
    q = untile(qt, K, N)
    want = np.zeros((M, N), np.float32)
    O.lib().orc_gemv_i8w(O.ORC_F16, O._p(q), O._p(s), O._p(x), M, K, N, O._p(want))
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 2e-3 * np.abs(want) + 2e-3 * np.abs(want).max(axis=1, keepdims=True)), err.max()
    if K * N <= 1 << 22:
        xf = O.f16_bits_to_f32(x).astype(np.float64)
        prod = xf @ q.T.astype(np.float64)
        bound = (K * 2.0 ** -24 * (np.abs(xf) @ np.abs(q.T.astype(np.float64))) + 2.0 ** -24 * np.abs(prod)) * s
        assert np.all(np.abs(got - prod * s) <= bound + 2.0 ** -24 * np.abs(prod * s))


def test_head_quantised_by_the_reference_retiles_bitwise():
    """A head quantised by the reference's own quantise_int8_tiled (lm_head_int8.cc, in its
    int8_tiled_index layout; compiled into oracle/_ref) re-tiled on the device by
    mi_i8w_from_ref_tiles: every byte equals this library's own quantisation of the same head
    in mi_i8w_index's layout, the scales are bitwise the same, and the GEMV over the re-tiled
    head is bitwise the GEMV over the library's own."""
    K, N, M = 512, 1024, 2
    rng = np.random.default_rng(19)
    w16 = O.f32_to_bf16_bits((0.05 * rng.standard_normal((N, K))).astype(np.float32))
    w16[7] = 0  # a zero row: s = 0, q = 0
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref is not built (python __graft_entry__.py builds it where /root/reference is)")
    q_ref = np.zeros(K * N, np.int8)
    s_ref = np.zeros(N, np.float32)
    R.ref_quantise_int8_tiled(O._p(w16), K, N, O._p(q_ref), O._p(s_ref))
    q_own = np.zeros(K * N, np.int8)
    s_own = np.zeros(N, np.float32)
    mi.check(mi.lib().mi_lm_head_int8_quantise(O._p(np.ascontiguousarray(O.bf16_bits_to_f32(w16))), K, N,
                                                 O._p(q_own), O._p(s_own)), "quantise")
    assert np.array_equal(s_ref.view(np.uint32), s_own.view(np.uint32))
    dref = dev(q_ref)
    dq = empty((K * N,), np.int8)
    mi.call("mi_i8w_from_ref_tiles", ptr(dref), K, N, ptr(dq), stream())
    sync()
    assert np.array_equal(host(dq, np.int8), q_own)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    dx, ds = dev(x), dev(s_ref)
    a, b = empty((M, N), np.float32), empty((M, N), np.float32)
    mi.call("mi_gemv_i8w", ptr(dq), ptr(ds), ptr(dx), ptr(a), M, K, N, stream())
    dq_own, ds_own = dev(q_own), dev(s_own)  # (held: a temporary's memory could be reused at once)
    mi.call("mi_gemv_i8w", ptr(dq_own), ptr(ds_own), ptr(dx), ptr(b), M, K, N, stream())
    sync()
    assert np.array_equal(host(a, np.uint32), host(b, np.uint32))
