"""The RMSNorm split across two GEMV launches: a RESID launch that writes only the residual and
its 64-column tiles' sums of squares (sums_out), and a launch that reads that residual with
the sums (in_sums) and forms the norm itself. The contract is bitwise: the second launch's
output equals the same launch on the x_next that the whole RESID epilogue writes (the
reference's res_norm chain, capture.cc:997, prep_res_fold + prep_norm_finish), for the
PARTIALS, SILU and QKV kinds, f16 and bf16 activations, 1 to 16 rows."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
EMPTY = 0xFFFFFFFF


def rand_w(K, N, seed):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, size=(K // 64, N)).astype(np.float32))
    return qw, sc


def handoff(n):
    d = empty((n,), np.float32)
    mi.call("mi_gemv_handoff_init", ptr(d), n, stream())
    return d


def bits16(v, act):
    return O.f32_to_f16_bits(v) if act == 0 else O.f32_to_bf16_bits(v)


class Residual:
    """One o-like RESID launch over [M][H] in both forms on the same inputs: the whole
    epilogue (resid, x_next) and the split one (resid, sums_out)."""

    def __init__(self, M, H, act, seed):
        K1, S1 = 1024, 4
        rng = np.random.default_rng(seed)
        qw, sc = rand_w(K1, H, seed)
        x1 = O.f32_to_f16_bits(rng.standard_normal((M, K1)).astype(np.float32))
        r0 = bits16(rng.standard_normal((M, H)).astype(np.float32) * 4, act)
        self.w = (1 + 0.05 * rng.standard_normal(H)).astype(np.float32)
        self.dw = dev(self.w)
        self.M, self.H, self.act = M, H, act
        dq, ds, dx = dev(qw), dev(sc), dev(x1)
        G = H // 64
        # whole: x_next
        self.dr_full, dss, drs = dev(r0), handoff(G * M * G), empty((M,), np.float32)
        self.dxn = empty((M, H), np.uint16)
        ep = mi.GemvEpilogue(kind=mi.EPI_RESID, resid=ptr(self.dr_full), sumsq=ptr(dss), rstd=ptr(drs),
                             next_norm_w=ptr(self.dw), x_next=ptr(self.dxn), eps=1e-6, act=act)
        h1, h2 = handoff(S1 * M * H), handoff(S1 * M * H)
        mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(dx), ptr(h1), M, K1, H, S1, C.byref(ep), stream())
        # split: sums_out
        self.dr, self.dsum = dev(r0), empty((M * G + M,), np.float32)
        ep = mi.GemvEpilogue(kind=mi.EPI_RESID, resid=ptr(self.dr), sums_out=ptr(self.dsum), eps=1e-6, act=act)
        mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(dx), ptr(h2), M, K1, H, S1, C.byref(ep), stream())
        sync()
        self.keep = (dq, ds, dx, dss, drs, h1, h2)

    def norm_in(self, ep):
        ep.in_sums = ptr(self.dsum)
        ep.in_norm_w = ptr(self.dw)
        ep.in_eps = 1e-6
        ep.act = self.act
        return ep


@pytest.mark.parametrize("M,act", [(1, 0), (3, 0), (8, 0), (16, 0), (1, 1), (4, 1)])
def test_sums_out_is_the_whole_epilogues_residual_and_sums(M, act):
    print(f"split resid M={M} act={act}", flush=True)
    R = Residual(M, 1024, act, 7 + M)
    assert np.array_equal(host(R.dr, np.uint16), host(R.dr_full, np.uint16))
    # the sums give the whole epilogue's x_next (sequential fp32 sum over tiles, then the norm)
    r = host(R.dr, np.uint16)
    sums = host(R.dsum, np.float32)[:M * (R.H // 64)].reshape(M, R.H // 64)
    assert np.all(host(R.dsum, np.uint32)[M * (R.H // 64):] == EMPTY)
    rf = O.f16_bits_to_f32(r) if act == 0 else O.bf16_bits_to_f32(r)
    for m in range(M):
        tot = np.float32(0)
        for g in range(R.H // 64):
            tot = np.float32(tot + sums[m, g])
            # each tile's sum is the 64-lane tree's; check it against fp64 closely
            ex = np.sum(rf[m, 64 * g:64 * g + 64].astype(np.float64) ** 2)
            assert abs(sums[m, g] - ex) <= 1e-5 * ex + 1e-30
        rstd = np.float32(1) / np.sqrt(np.float32(tot / np.float32(R.H) + np.float32(1e-6)))
        xn = O.f16_bits_to_f32(host(R.dxn, np.uint16)[m])
        want = (rf[m] * rstd).astype(np.float32) * R.w
        assert np.allclose(xn, want, rtol=2 ** -7 if act else 2 ** -10, atol=1e-6)


@pytest.mark.parametrize("M,act,S", [(1, 0, 2), (3, 0, 4), (16, 0, 2), (1, 1, 2), (8, 1, 4)])
def test_norm_in_partials_bitwise(M, act, S):
    print(f"norm_in partials M={M} act={act} S={S}", flush=True)
    R = Residual(M, 1024, act, 30 + M)
    K, N = R.H, 512
    qw, sc = rand_w(K, N, 40 + M)
    dq, ds = dev(qw), dev(sc)
    want = empty((S, M, N), np.float32)
    mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(R.dxn), ptr(want), M, K, N, S, stream())
    G = K // 64
    for rep in range(2):  # the first launch forms the rows' rstd and leaves it after the sums
        got = empty((S, M, N), np.float32)
        ep = R.norm_in(mi.GemvEpilogue(kind=mi.EPI_PARTIALS))
        mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(R.dr), ptr(got), M, K, N, S, C.byref(ep), stream())
        sync()
        assert np.array_equal(host(got, np.uint32), host(want, np.uint32)), rep
        assert not np.any(host(R.dsum, np.uint32)[M * G:] == EMPTY), rep


@pytest.mark.parametrize("M,act", [(1, 0), (4, 0), (16, 0), (1, 1)])
def test_norm_in_silu_bitwise(M, act):
    print(f"norm_in silu M={M} act={act}", flush=True)
    R = Residual(M, 1024, act, 50 + M)
    K, I, S = R.H, 768, 4
    N = 2 * I
    qw, sc = rand_w(K, N, 60 + M)
    dq, ds = dev(qw), dev(sc)
    outs = []
    for ni in (False, True):
        dh = empty((M, I), np.uint16)
        ep = mi.GemvEpilogue(kind=mi.EPI_SILU, h=ptr(dh), act=act)
        if ni:
            R.norm_in(ep)
        hp = handoff(S * M * N)
        mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(R.dr if ni else R.dxn), ptr(hp), M, K, N, S,
                C.byref(ep), stream())
        sync()
        outs.append(host(dh, np.uint16).copy())
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("M,act", [(1, 0), (3, 0), (1, 1)])
def test_norm_in_qkv_bitwise(M, act):
    QH, KVH, HD, S = 16, 2, 128, 4
    print(f"norm_in qkv M={M} act={act}", flush=True)
    R = Residual(M, 1024, act, 70 + M)
    sh = O.attn_shape(QH, KVH, HD, rot_dim=HD)
    msh = mi.lib_shape(sh, act)
    K, N, pos, Lm = R.H, sh.qkv_n, 300, 512
    rng = np.random.default_rng(M)
    qw, sc = rand_w(K, N, 80 + M)
    dq, ds = dev(qw), dev(sc)
    qn = dev((1 + 0.05 * rng.standard_normal(HD)).astype(np.float32))
    kn = dev((1 + 0.05 * rng.standard_normal(HD)).astype(np.float32))
    rope = dev(O.rope_table(1e6, HD, Lm))
    kk = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    outs = []
    for ni in (False, True):
        c = np.zeros(64, np.uint32)
        c[0], c[1] = pos, M
        dc, aq, k2, v2 = dev(c), empty((M, QH, HD), np.float32), dev(kk), dev(kk)
        aq.zero_()
        ep = mi.GemvEpilogue(kind=mi.EPI_QKV, ctrl=ptr(dc), shape=C.cast(C.pointer(msh), C.c_void_p),
                             q_norm=ptr(qn), k_norm=ptr(kn), rope=ptr(rope), attn_q=ptr(aq), kv_k=ptr(k2),
                             kv_v=ptr(v2), row_stride=HD, head_stride=Lm * HD, kv_len=Lm, act=act)
        if ni:
            R.norm_in(ep)
        hp = handoff(S * M * N)
        mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(R.dr if ni else R.dxn), ptr(hp), M, K, N, S,
                C.byref(ep), stream())
        sync()
        outs.append((host(aq, np.uint32).copy(), host(k2, np.uint16).copy(), host(v2, np.uint16).copy()))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_split_norm_refusals():
    qw, sc = rand_w(1024, 512, 1)
    dq, ds, dx = dev(qw), dev(sc), dev(np.zeros((1, 1024), np.uint16))
    dpart, dsum = handoff(4 * 512), empty((1, 17), np.float32)
    # in_sums without weights; with the RESID / LOGITS kinds; more than 8 k-groups per slice
    for ep, S in ((mi.GemvEpilogue(kind=mi.EPI_PARTIALS, in_sums=ptr(dsum)), 4),
                  (mi.GemvEpilogue(kind=mi.EPI_RESID, resid=ptr(dx), sums_out=ptr(dsum), in_sums=ptr(dsum),
                                   in_norm_w=ptr(dsum)), 4),
                  (mi.GemvEpilogue(kind=mi.EPI_PARTIALS, in_sums=ptr(dsum), in_norm_w=ptr(dsum)), 1)):
        rc = mi.lib().mi_gemv_w4a16_ex(ptr(dq), ptr(ds), ptr(dx), ptr(dpart), 1, 1024, 512, S, C.byref(ep), stream())
        assert rc != 0
