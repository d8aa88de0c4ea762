"""W4A16 GEMV / small-M GEMM on the GPU, through the C ABI, against the CPU oracle.

Bars (the reference's gemm_sm_test / gemv_test): unpack bit-exact; every output within
the N2 bound 2^-16 * sum|w x| of the fp64 reference (tests/kernels/gemm_sm_ref.h:180-225);
bit-exact where every operation is exact; property R (row m independent of M); replays
bitwise."""
import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu


def rand_w(K, N, seed, lo=0.002, hi=0.02):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(lo, hi, size=(K // 64, N)).astype(np.float32))
    return qw, sc


def run_gemv(qw, sc, x16, K, N, S):
    M = x16.shape[0]
    dq, ds, dx = dev(qw), dev(sc), dev(x16)
    part = empty((S, M, N), np.float32)
    print(f"gemv M={M} K={K} N={N} S={S}", flush=True)
    mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(part), M, K, N, S, stream())
    sync()
    return host(part, np.float32)


def test_int4_dequant_bit_exact():
    K, N = 512, 320
    qw, sc = rand_w(K, N, 1)
    sc[0, :8] = [0x0001, 0x03FF, 0x8001, 0x0400, 0x7BFF, 0x3C00, 0xBC00, 0x0000]  # subnormals, extremes
    dq, ds = dev(qw), dev(sc)
    out = empty((K, N), np.float32)
    mi.call("mi_int4_dequant", ptr(dq), ptr(ds), ptr(out), K, N, stream())
    sync()
    want = O.int4_dequant(qw, sc, K, N)
    assert np.array_equal(host(out, np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("K,N", [(4096, 4096), (512, 192), (17408 // 4, 320)])
def test_gemv_n2_bound(M, K, N):
    qw, sc = rand_w(K, N, K + N + M)
    x16 = O.f32_to_f16_bits(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    S = mi.lib().mi_gemv_pick_s(K, N)
    part = run_gemv(qw, sc, x16, K, N, S)
    got = np.zeros((M, N), np.float32)
    for s in range(S):
        got = got + part[s]
    ref, bound = O.gemv_ref(qw, sc, K, N, O.f16_bits_to_f32(x16))
    over, mr = O.n2_over(got, ref, bound)
    assert over == 0, f"N2 violated: max ratio {mr}"
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(ref) + 2e-3 * np.abs(ref).max())


@pytest.mark.parametrize("S", [1, 2, 8, 64])
def test_gemv_every_split(S):
    K, N, M = 4096, 128, 1
    qw, sc = rand_w(K, N, 77)
    x16 = O.f32_to_f16_bits(np.random.default_rng(3).standard_normal((M, K)).astype(np.float32))
    part = run_gemv(qw, sc, x16, K, N, S)
    ref, bound = O.gemv_ref(qw, sc, K, N, O.f16_bits_to_f32(x16))
    got = part.sum(axis=0, dtype=np.float32)
    assert O.n2_over(got, ref, bound)[0] == 0


def test_gemv_exact_arithmetic_bitwise():
    """Integer activations, power-of-two scales: every product and partial sum is exact,
    so the device result equals the integer dot product bit for bit - pins nibble order,
    k-group index, column mapping and the pair permutation of the activations."""
    K, N = 1024, 256
    rng = np.random.default_rng(9)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = rng.choice(np.array([0x3C00, 0x3800, 0x4000, 0x3400], np.uint16), size=(K // 64, N))
    for M in (1, 3, 16):
        x = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
        x16 = O.f32_to_f16_bits(x)
        exact = x.astype(np.float64) @ O.int4_dequant(qw, sc, K, N).astype(np.float64)
        for S in (1, 4):
            part = run_gemv(qw, sc, x16, K, N, S)
            got = part.sum(axis=0, dtype=np.float64)
            assert np.array_equal(got, exact)


def test_gemv_property_r_and_replay():
    """Row m's bits do not depend on M or on the other rows (gemm_sm.cl:36-41), and two
    launches give the same bits."""
    K, N = 2048, 512
    qw, sc = rand_w(K, N, 5)
    S = mi.lib().mi_gemv_pick_s(K, N)
    x16 = O.f32_to_f16_bits(np.random.default_rng(11).standard_normal((16, K)).astype(np.float32))
    full = run_gemv(qw, sc, x16, K, N, S)
    again = run_gemv(qw, sc, x16, K, N, S)
    assert np.array_equal(full.view(np.uint32), again.view(np.uint32))
    for M in (1, 4, 8):
        for m0 in (0, 16 - M):
            sub = run_gemv(qw, sc, np.ascontiguousarray(x16[m0:m0 + M]), K, N, S)
            assert np.array_equal(sub.view(np.uint32), full[:, m0:m0 + M].view(np.uint32))


def test_cfg1_gemv_fp16_out():
    """x[4096] ~N(0,1) fp16, uniform nibbles, scales ~U(0.002, 0.02),
    K = N = 4096, fp32 accumulate, fp16 out; against the reference's fp32 twin
    (gemv.cl's order) within rel 2e-3 and against fp64 within N2."""
    K = N = 4096
    qw, sc = rand_w(K, N, 1234)
    x16 = O.f32_to_f16_bits(np.random.default_rng(1234).standard_normal((1, K)).astype(np.float32))
    S = mi.lib().mi_gemv_pick_s(K, N)
    dq, ds, dx = dev(qw), dev(sc), dev(x16)
    part = empty((S, 1, N), np.float32)
    out = empty((1, N), np.uint16)
    mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(part), 1, K, N, S, stream())
    mi.call("mi_fold_partials", ptr(part), ptr(out), None, S, 1, N, stream())
    sync()
    y = O.f16_bits_to_f32(host(out, np.uint16))[0].astype(np.float64)
    xf = O.f16_bits_to_f32(x16)
    twin = O.gemv_twin(qw, sc, K, N, xf, S=1)[0].astype(np.float64)
    ref, bound = O.gemv_ref(qw, sc, K, N, xf)
    assert np.all(np.abs(y - twin) <= 2e-3 * np.abs(twin) + 1e-3 * np.abs(twin).max())
    # fp16 output: N2 widened by the final fp16 rounding (half an ulp of the result)
    assert np.all(np.abs(y - ref[0]) <= np.ldexp(bound[0], -16) + np.abs(ref[0]) * 2.0 ** -11 + 1e-7)
