"""GQA decode attention on the GPU (fp16 and int8 KV, contiguous and paged) vs the oracle.

Bars: softmax attention within rel 2e-3 of the fp64 reference (the reference holds its
readers to the fp64 attend by cosine, tests/kernels/kv8_ref.h:1-12) and of the oracle's
restatement of attn_decode_v2's order; cosine >= 0.99999; KV paging bitwise equal to the
contiguous cache (attn_v2.cl:123-131); row m of an M-row step bitwise the 1-row step at
pos + m; replays bitwise."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16
L = O.lib


def ctrl_dev(pos, n_act):
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos, n_act
    return dev(c)


def make_kv(kind, KVH, Lm, HD, seed):
    rng = np.random.default_rng(seed)
    if kind == 0:
        k = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
        v = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
        return k, v, None, None
    k = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    v = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    ks = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    vs = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    return k, v, ks, vs


def gpu_attention(sh, q, kind, k, v, ks, vs, pos, M, tgt, pages=None, page=0, n_act=None):
    HD, QH = sh.head_dim, sh.q_heads
    Lm = k.shape[1]
    print(f"attn kind={kind} HD={HD} QH={QH} pos={pos} M={M} tgt={tgt} paged={pages is not None}", flush=True)
    ctrl = ctrl_dev(pos, M if n_act is None else n_act)
    part = empty((QH, tgt, M, HD + 2), np.float32)
    out = dev(np.full((M, QH * HD), 0xFFFF, np.uint16))
    dk, dv, dks, dvs, dq = dev(k), dev(v), dev(ks), dev(vs), dev(q)
    dpg = dev(pages)
    shp = mi.shape_ref(sh)
    mi.call("mi_attn_decode", ptr(ctrl), ptr(dq), kind, ptr(dk), ptr(dv), ptr(dks), ptr(dvs), HD, Lm * HD,
            1, Lm, ptr(dpg), page, Lm, ptr(part), M, tgt, shp, stream())
    mi.call("mi_attn_reduce", ptr(ctrl), ptr(part), None, ptr(out), M, tgt, Lm, shp, stream())
    sync()
    return host(out, np.uint16), host(part, np.float32)


def fp64_attention(sh, q, kind, k, v, ks, vs, n, pages=None, page=0):
    HD, QH, G = sh.head_dim, sh.q_heads, sh.q_heads // sh.kv_heads
    Lm = k.shape[1]
    o = np.zeros((QH, HD))
    for h in range(QH):
        L().orc_attend64(C.byref(sh), O._p(np.ascontiguousarray(q[h])), h // G, n, kind, F16, O._p(k), O._p(v),
                         O._p(ks), O._p(vs), HD, Lm * HD, 1, Lm, O._p(pages), page, O._p(o[h]))
    return o


def check_close(got16, want, rtol=2e-3):
    g = O.f16_bits_to_f32(got16).astype(np.float64).reshape(want.shape)
    err = np.abs(g - want)
    assert np.all(err <= rtol * np.abs(want) + 2e-3 * np.abs(want).max(axis=-1, keepdims=True)), err.max()
    cos = (g * want).sum(-1) / np.sqrt((g * g).sum(-1) * (want * want).sum(-1))
    assert cos.min() >= 0.99999


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("QH,KVH,HD", [(40, 8, 128), (16, 2, 256)])
@pytest.mark.parametrize("pos", [0, 77, 4095])
def test_decode_vs_fp64_and_oracle(kind, QH, KVH, HD, pos):
    Lm, tgt = 4096, 128
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(kind, KVH, Lm, HD, pos + HD)
    q = np.random.default_rng(pos).standard_normal((1, QH, HD)).astype(np.float32)
    got, _ = gpu_attention(sh, q, kind, k, v, ks, vs, pos, 1, tgt)
    want = fp64_attention(sh, q[0], kind, k, v, ks, vs, pos + 1)
    check_close(got[0].reshape(QH, HD), want)
    # the oracle's restatement of attn_decode_v2 + attn_reduce_v2 at the same grid
    part = np.zeros((QH, tgt, 1, HD + 2), np.float32)
    L().orc_attn_decode_v2(F16, C.byref(sh), pos, 1, 1, tgt, O._p(q), kind, O._p(k), O._p(v), O._p(ks),
                           O._p(vs), HD, Lm * HD, 1, Lm, None, 0, O._p(part))
    ref = np.zeros((1, QH * HD), np.uint16)
    L().orc_attn_reduce_v2(F16, C.byref(sh), pos, 1, 1, tgt, O._p(part), None, O._p(ref))
    check_close(got[0].reshape(QH, HD), O.f16_bits_to_f32(ref[0]).astype(np.float64).reshape(QH, HD))


@pytest.mark.parametrize("QH,KVH,HD", [(8, 8, 128), (8, 4, 128), (8, 2, 128), (12, 2, 128), (16, 2, 256),
                                      (8, 2, 256)])
@pytest.mark.parametrize("Lm,tgt,pos", [(512, 4, 300), (512, 4, 45), (4096, 128, 3000)])
def test_decode_every_gqa_and_block_length(QH, KVH, HD, Lm, tgt, pos):
    """Every GQA ratio the kernel instantiates, blocks of one and of several 16-position
    chunks per wave (tgt 4 at 512 cached rows: the double-buffered variant), partial blocks."""
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(0, KVH, Lm, HD, pos + QH)
    q = np.random.default_rng(pos + KVH).standard_normal((1, QH, HD)).astype(np.float32)
    got, _ = gpu_attention(sh, q, 0, k, v, ks, vs, pos, 1, tgt)
    want = fp64_attention(sh, q[0], 0, k, v, ks, vs, pos + 1)
    check_close(got[0].reshape(QH, HD), want)


@pytest.mark.parametrize("kind", [0, 1])
def test_long_context_paged_bitwise(kind):
    """BASELINE config 3 shape (40 q / 8 kv, hd 128) at L = 32768, 64-token pages in a
    shuffled table: the paged cache gives the same bits as the contiguous one."""
    QH, KVH, HD, Lm, P, tgt = 40, 8, 128, 32768, 64, 128
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(kind, KVH, Lm, HD, 7)
    q = np.random.default_rng(8).standard_normal((1, QH, HD)).astype(np.float32)
    pos = Lm - 1
    a, pa = gpu_attention(sh, q, kind, k, v, ks, vs, pos, 1, tgt)
    rng = np.random.default_rng(9)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    phys = np.concatenate([np.arange(pg * P, pg * P + P) for pg in pages])
    kp, vp = np.empty_like(k), np.empty_like(v)
    kp[:, phys], vp[:, phys] = k, v
    ksp = vsp = None
    if kind:
        ksp, vsp = np.empty_like(ks), np.empty_like(vs)
        ksp[:, phys], vsp[:, phys] = ks, vs
    b, pb = gpu_attention(sh, q, kind, kp, vp, ksp, vsp, pos, 1, tgt, pages, P)
    assert np.array_equal(a, b)
    assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32))
    # and against fp64 for a few heads (the full fp64 pass over 32k keys is slow on the host)
    want = fp64_attention(sh, q[0], kind, k, v, ks, vs, pos + 1)
    check_close(a[0].reshape(QH, HD), want)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("QH,KVH,HD", [(40, 8, 128), (16, 2, 256), (8, 1, 128)])
@pytest.mark.parametrize("Lm,tgt,pos,P", [(4096, 8, 4095, 64), (4096, 16, 2000, 32), (1024, 4, 1000, 16)])
def test_decode_ring_paths_paged(kind, QH, KVH, HD, Lm, tgt, pos, P):
    """The decode kernel's LDS ring at several groups per wave (blocks of 512 / 256 / 320
    positions: the ring's slots reused, pairs of groups per softmax step, a wave's odd last
    group, a partial last group), paged with a shuffled table of 64-, 32- and 16-position
    pages, f16 and int8 rows of 128 and 256: bitwise the contiguous cache, and within rel 2e-3
    of the fp64 reference."""
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(kind, KVH, Lm, HD, pos + HD + kind)
    q = np.random.default_rng(pos + QH).standard_normal((1, QH, HD)).astype(np.float32)
    a, pa = gpu_attention(sh, q, kind, k, v, ks, vs, pos, 1, tgt)
    rng = np.random.default_rng(P + kind)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    phys = np.concatenate([np.arange(pg * P, pg * P + P) for pg in pages])
    kp, vp = np.empty_like(k), np.empty_like(v)
    kp[:, phys], vp[:, phys] = k, v
    ksp = vsp = None
    if kind:
        ksp, vsp = np.empty_like(ks), np.empty_like(vs)
        ksp[:, phys], vsp[:, phys] = ks, vs
    b, pb = gpu_attention(sh, q, kind, kp, vp, ksp, vsp, pos, 1, tgt, pages, P)
    assert np.array_equal(a, b)
    want = fp64_attention(sh, q[0], kind, k, v, ks, vs, pos + 1)
    check_close(a[0].reshape(QH, HD), want)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("QH,KVH,HD", [(40, 8, 128), (16, 2, 256), (8, 8, 128), (8, 2, 128), (8, 4, 128),
                                      (12, 2, 128)])
@pytest.mark.parametrize("Lm,tgt,pos,M,n_act", [
    (4096, 128, 2045, 4, 4),   # one block size, 4 rows
    (512, 4, 252, 8, 8),       # the block size changes at row 4 (ppw 64 -> 128)
    (512, 4, 250, 16, 13),     # 16 rows, 13 live, the change at row 6
    (1024, 8, 700, 3, 3),      # several groups per wave, rows ending inside the last group
    (1024, 8, 761, 7, 7),      # rows whose last block is new to the later rows
])
def test_rows_are_bitwise_their_single_row_steps(kind, QH, KVH, HD, Lm, tgt, pos, M, n_act):
    """Several rows per work-group (16 / GQA rows' heads in the product columns): every live
    row's output and partials bitwise the one-row launch at pos + m; replays bitwise; rows past
    n_act untouched."""
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(kind, KVH, Lm, HD, 3 + kind)
    q = np.random.default_rng(4 + M).standard_normal((M, QH, HD)).astype(np.float32)
    full, pf = gpu_attention(sh, q, kind, k, v, ks, vs, pos, M, tgt, n_act=n_act)
    for m in range(n_act):
        one, p1 = gpu_attention(sh, np.ascontiguousarray(q[m:m + 1]), kind, k, v, ks, vs, pos + m, 1, tgt)
        assert np.array_equal(one[0], full[m]), m
        nb = (pos + m) // mi.lib().mi_attn_ppw(pos + m + 1, tgt) + 1
        assert np.array_equal(p1[:, :nb, 0].view(np.uint32), pf[:, :nb, m].view(np.uint32)), m
    assert np.all(full[n_act:] == 0xFFFF)
    again, _ = gpu_attention(sh, q, kind, k, v, ks, vs, pos, M, tgt, n_act=n_act)
    assert np.array_equal(full, again)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("QH,KVH,HD", [(40, 8, 128), (16, 2, 256)])
def test_rows_paged_bitwise_contiguous(kind, QH, KVH, HD):
    """Several rows per work-group over a paged cache (32-position pages, shuffled table):
    bitwise the contiguous cache, and each row bitwise its one-row launch."""
    Lm, tgt, pos, M, P = 1024, 8, 761, 8, 32
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(kind, KVH, Lm, HD, 11 + kind)
    q = np.random.default_rng(12).standard_normal((M, QH, HD)).astype(np.float32)
    a, _ = gpu_attention(sh, q, kind, k, v, ks, vs, pos, M, tgt)
    rng = np.random.default_rng(13)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    phys = np.concatenate([np.arange(pg * P, pg * P + P) for pg in pages])
    kp, vp = np.empty_like(k), np.empty_like(v)
    kp[:, phys], vp[:, phys] = k, v
    ksp = vsp = None
    if kind:
        ksp, vsp = np.empty_like(ks), np.empty_like(vs)
        ksp[:, phys], vsp[:, phys] = ks, vs
    b, _ = gpu_attention(sh, q, kind, kp, vp, ksp, vsp, pos, M, tgt, pages, P)
    assert np.array_equal(a, b)
    for m in (0, M - 1):
        one, _ = gpu_attention(sh, np.ascontiguousarray(q[m:m + 1]), kind, kp, vp, ksp, vsp, pos + m, 1, tgt,
                               pages, P)
        assert np.array_equal(one[0], b[m]), m


def test_reduce_matches_oracle_merge_on_device_partials():
    """attn_reduce_v2's merge on the GPU's own partials: within 1 fp16 ulp of the oracle's
    sequential merge (the device forms the same sum with a common max; exp differs by <= 1
    ulp)."""
    QH, KVH, HD, Lm, tgt = 40, 8, 128, 8192, 32
    sh = O.attn_shape(QH, KVH, HD)
    k, v, ks, vs = make_kv(0, KVH, Lm, HD, 5)
    q = np.random.default_rng(6).standard_normal((1, QH, HD)).astype(np.float32)
    pos = 6000
    got, part = gpu_attention(sh, q, 0, k, v, ks, vs, pos, 1, tgt)
    ref = np.zeros((1, QH * HD), np.uint16)
    L().orc_attn_reduce_v2(F16, C.byref(sh), pos, 1, 1, tgt, O._p(np.ascontiguousarray(part)), None, O._p(ref))
    a = O.f16_bits_to_f32(got).astype(np.float64)
    b = O.f16_bits_to_f32(ref).astype(np.float64)
    assert np.all(np.abs(a - b) <= np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10 * 1.01)


@pytest.mark.parametrize("QH,KVH,HD,rot,gated,qk,paged,M,n_act,pos,tgt", [
    (40, 8, 128, 128, False, True, False, 1, 1, 4096, 64),
    (40, 8, 128, 128, False, False, True, 4, 3, 2045, 32),
    (16, 2, 256, 256, False, True, False, 2, 2, 700, 128),
    (24, 4, 256, 64, True, True, True, 3, 3, 130, 8),
    (8, 8, 128, 64, False, True, False, 8, 8, 63, 16),
])
def test_prep_decode_fused_is_prep_then_decode(QH, KVH, HD, rot, gated, qk, paged, M, n_act, pos, tgt):
    """mi_attn_prep_decode against mi_attn_prep followed by mi_attn_decode on the same inputs:
    the partials of every active row, the whole cache (each new K/V row written once, nothing
    else touched) and the gate, bit for bit."""
    sh = O.attn_shape(QH, KVH, HD, rot_dim=rot, gated=gated)
    Lm, S, P = 4224, 3, 64
    rng = np.random.default_rng(pos + M)
    part = rng.standard_normal((S, M, sh.qkv_n)).astype(np.float32)
    qn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk else None
    kn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk else None
    rope = O.rope_table(1e6, rot, Lm)
    pages = rng.permutation(Lm // P).astype(np.uint32) if paged else None
    kk = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    vv = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    print(f"prep_decode QH={QH} KVH={KVH} HD={HD} rot={rot} gated={gated} M={M} n={n_act} pos={pos}", flush=True)
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos, n_act
    keep = [dev(part), dev(qn), dev(kn), dev(rope), dev(pages)]
    shp = mi.shape_ref(sh)
    outs = []
    for fused in (False, True):
        ctrl = dev(c)
        dk, dv = dev(kk), dev(vv)
        dq = empty((M, QH, HD), np.float32)
        dg = empty((M, QH, HD), np.float32)
        dg.zero_()
        dp = empty((QH, tgt, M, HD + 2), np.float32)
        dp.zero_()
        if fused:
            mi.call("mi_attn_prep_decode", ptr(ctrl), ptr(keep[0]), S, M, shp, ptr(keep[1]), ptr(keep[2]),
                    ptr(keep[3]), ptr(dg), ptr(dk), ptr(dv), HD, Lm * HD, ptr(keep[4]), P if paged else 0, Lm,
                    ptr(dp), tgt, stream())
        else:
            mi.call("mi_attn_prep", ptr(ctrl), ptr(keep[0]), S, M, shp, ptr(keep[1]), ptr(keep[2]), ptr(keep[3]),
                    ptr(dq), ptr(dg), ptr(dk), ptr(dv), HD, Lm * HD, ptr(keep[4]), P if paged else 0, Lm, stream())
            mi.call("mi_attn_decode", ptr(ctrl), ptr(dq), 0, ptr(dk), ptr(dv), None, None, HD, Lm * HD, 0, 0,
                    ptr(keep[4]), P if paged else 0, Lm, ptr(dp), M, tgt, shp, stream())
        sync()
        outs.append((host(dp, np.uint32), host(dk, np.uint16), host(dv, np.uint16), host(dg, np.uint32),
                     host(ctrl, np.uint32)))
    (p0, k0, v0, g0, c0), (p1, k1, v1, g1, c1) = outs
    for m in range(n_act):
        L = pos + m + 1
        nb = (L - 1) // O.lib().orc_v2_ppw(L, tgt) + 1
        nb = min(nb, tgt)
        assert np.array_equal(p0[:, :nb, m], p1[:, :nb, m]), m
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    assert not np.array_equal(k0, kk)  # the new rows were written
    if gated:
        assert np.array_equal(g0[:n_act], g1[:n_act])
    assert c0[18] == c1[18] == 0
