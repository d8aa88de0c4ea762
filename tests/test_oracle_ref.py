"""The oracle against the reference's OWN scalar twins, compiled from /root/reference into
oracle/_ref/libref.so by oracle/build_oracle.py. Under bf16 activations and the reference's
shapes the oracle must reproduce them bit for bit. CPU only; skipped when the reference
build is absent."""
import ctypes as C

import numpy as np
import pytest

import oracle as O

R = O.ref()
L = O.lib
pytestmark = pytest.mark.skipif(R is None, reason="oracle/_ref not built (needs /root/reference)")
BF = O.ORC_BF16
P = O._p


def bits(a):
    return np.asarray(a).view(np.uint32 if np.asarray(a).dtype == np.float32 else np.uint16)


def test_conversions():
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(5000) * 10.0 ** rng.integers(-8, 6, 5000)).astype(np.float32)
    for v in vals:
        assert L().orc_f32_to_bf16(float(v)) == R.ref_f32_to_bf16(float(v))
        assert L().orc_f32_to_f16_ftz(float(v)) == R.ref_f32_to_f16(float(v))
        assert L().orc_f32_to_f16_sat(float(v)) == R.ref_kv8_f32_to_f16_rne(float(v))
    for h in range(0, 65536, 7):
        a, b = L().orc_f16_to_f32(h), R.ref_f16_to_f32(h)
        assert (np.isnan(a) and np.isnan(b)) or a == b


def _rand(K, N, seed):
    qw = np.zeros((K // 8, N), np.uint32)
    sc = np.zeros((K // 64, N), np.uint16)
    R.ref_int4_random(K, N, seed, P(qw), P(sc))
    return qw, sc


def test_int4_dequant_and_layouts():
    K, N = 256, 64
    qw, sc = _rand(K, N, 5)
    a = np.zeros((K, N), np.float32)
    b = np.zeros((K, N), np.float32)
    L().orc_int4_dequant(P(qw), P(sc), K, N, P(a))
    R.ref_int4_dequant(P(qw), P(sc), K, N, P(b))
    assert np.array_equal(bits(a), bits(b))
    t1 = np.zeros((N // 16) * (K // 64) * 136, np.uint32)
    t2 = np.zeros_like(t1)
    L().orc_repack_layout1(P(qw), P(sc), K, N, P(t1))
    R.ref_repack_layout1(P(qw), P(sc), K, N, P(t2))
    assert np.array_equal(t1, t2)
    qb, sb = _rand(K, N, 6)
    o1q = np.zeros((K // 8, 2 * N), np.uint32); o1s = np.zeros((K // 64, 2 * N), np.uint16)
    o2q = np.zeros_like(o1q); o2s = np.zeros_like(o1s)
    L().orc_interleave16_l0(P(qw), P(sc), P(qb), P(sb), K, N, P(o1q), P(o1s))
    R.ref_interleave16_l0(P(qw), P(sc), P(qb), P(sb), K, N, P(o2q), P(o2s))
    assert np.array_equal(o1q, o2q) and np.array_equal(o1s, o2s)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("S", [1, 2, 4, 8])
def test_gemv_twin_and_fp64(layout, S):
    K, N, M = 1024, 128, 3
    qw, sc = _rand(K, N, 17 + S)
    x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.random.default_rng(S).uniform(-1, 1, (M, K))))
    x = np.ascontiguousarray(x)
    words, scales = qw, sc
    if layout == 1:
        words = np.zeros((N // 16) * (K // 64) * 136, np.uint32)
        L().orc_repack_layout1(P(qw), P(sc), K, N, P(words))
        scales = None
    a = np.zeros((M, N), np.float32); b = np.zeros((M, N), np.float32)
    L().orc_gemv_twin(layout, P(words), P(scales), K, N, P(x), M, S, P(a))
    R.ref_twin_gemv(layout, P(words), P(scales), K, N, P(x), M, S, P(b))
    assert np.array_equal(bits(a), bits(b))
    ra = np.zeros((M, N)); ba = np.zeros((M, N)); rb = np.zeros((M, N)); bb = np.zeros((M, N))
    L().orc_gemv_ref(layout, P(words), P(scales), K, N, P(x), M, P(ra), P(ba))
    R.ref_gemv_ref(layout, P(words), P(scales), K, N, P(x), M, P(rb), P(bb))
    assert np.array_equal(ra, rb) and np.array_equal(ba, bb)


@pytest.mark.parametrize("S_PREV", [0, 1, 4])
def test_prep_res_norm_fold_finish(S_PREV):
    M, K, G = 2, 5120, 20
    rng = np.random.default_rng(S_PREV)
    part = np.ascontiguousarray((rng.standard_normal((max(S_PREV, 1), M, K)) * 0.5).astype(np.float32))
    resid = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = np.ascontiguousarray((1 + 0.02 * rng.standard_normal(K)).astype(np.float32))
    r1, r2 = resid.copy(), resid.copy()
    x1 = np.zeros((M, K), np.uint16); x2 = np.zeros((M, K), np.uint16)
    L().orc_res_norm(BF, P(part), P(r1), P(w), P(x1), M, K, S_PREV, 1e-6)
    R.ref_res_norm(P(part), P(r2), P(w), P(x2), M, K, S_PREV)
    assert np.array_equal(r1, r2) and np.array_equal(x1, x2)
    r1, r2 = resid.copy(), resid.copy()
    s1 = np.zeros((G, M), np.float32); s2 = np.zeros((G, M), np.float32)
    L().orc_res_fold(BF, P(part), P(r1), P(s1), M, K, S_PREV, G)
    R.ref_res_fold(P(part), P(r2), P(s2), M, K, S_PREV, G)
    assert np.array_equal(r1, r2) and np.array_equal(bits(s1), bits(s2))
    L().orc_norm_finish(BF, P(s1), P(r1), P(w), P(x1), M, K, G, 1e-6)
    R.ref_norm_finish(P(s2), P(r2), P(w), P(x2), M, K, G)
    assert np.array_equal(x1, x2)


def test_prep_silu_mul():
    S = R.ref_silu_s()
    M, N = 2, 1024
    part = np.ascontiguousarray((np.random.default_rng(3).standard_normal((S, M, 2 * N)) * 2).astype(np.float32))
    a = np.zeros((M, N), np.uint16); b = np.zeros((M, N), np.uint16)
    L().orc_silu_mul(BF, P(part), P(a), M, N, S)
    R.ref_silu_mul(P(part), P(b), M, N)
    assert np.array_equal(a, b)


# attn_ref's compiled shapes (tests/kernels/attn_ref.h:84-99)
QH, KVH, HD, ROT = 24, 4, 256, 64


def _qwen_shape():
    return O.attn_shape(QH, KVH, HD, rot_dim=ROT, gated=True)


def test_attn_prep_bitwise():
    sh = _qwen_shape()
    assert sh.qkv_n == 14336 and sh.k_off == 12288 and sh.v_off == 13312
    assert sh.scale == 0.0625
    M, n_act, pos, max_len = 2, 2, 41, 128
    rng = np.random.default_rng(8)
    part = np.ascontiguousarray(rng.standard_normal((2, M, sh.qkv_n)).astype(np.float32))
    fa_small = np.ascontiguousarray((1 + 0.05 * rng.standard_normal(512)).astype(np.float32))
    rope = O.rope_table(1e7, ROT, max_len)
    aq1 = np.zeros((M, QH, HD), np.float32); aq2 = np.zeros_like(aq1)
    g1 = np.zeros((M, QH, HD), np.float32); g2 = np.zeros_like(g1)
    k1 = np.zeros((max_len, KVH, HD), np.uint16); k2 = np.zeros_like(k1)
    v1 = np.zeros_like(k1); v2 = np.zeros_like(k1)
    L().orc_attn_prep(BF, C.byref(sh), pos, n_act, M, P(part), 2, P(fa_small), P(fa_small[256:].copy()),
                      P(rope), P(aq1), P(g1), P(k1), P(v1), KVH * HD, HD, None, 0)
    R.ref_attn_prep(pos, n_act, M, P(part), P(fa_small), P(rope), P(aq2), P(g2), P(k2), P(v2))
    assert np.array_equal(bits(aq1), bits(aq2))
    assert np.array_equal(bits(g1), bits(g2))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


@pytest.mark.parametrize("pos,n_act", [(0, 1), (63, 1), (64, 2), (700, 3), (1023, 1)])
def test_attn_decode_reduce_bitwise(pos, n_act):
    """v2 at tgt = max_len / 64 walks exactly v1's 64-position blocks (ppw = 64 while
    L <= 64 tgt), so the oracle's v2 must equal the reference's v1 twin bit for bit."""
    sh = _qwen_shape()
    M, max_len = 4, 1024
    tgt = max_len // 64
    assert all(O.lib().orc_v2_ppw(p + 1, tgt) == 64 for p in range(max_len))
    rng = np.random.default_rng(pos)
    q = np.ascontiguousarray(rng.standard_normal((M, QH, HD)).astype(np.float32))
    k = O.f32_to_bf16_bits(rng.standard_normal((max_len, KVH, HD)).astype(np.float32))
    v = O.f32_to_bf16_bits(rng.standard_normal((max_len, KVH, HD)).astype(np.float32))
    gate = np.ascontiguousarray(rng.standard_normal((M, QH, HD)).astype(np.float32))
    p1 = np.zeros((QH, tgt, M, HD + 2), np.float32)
    p2 = np.zeros_like(p1)
    L().orc_attn_decode_v2(BF, C.byref(sh), pos, n_act, M, tgt, P(q), 0, P(k), P(v), None, None,
                           KVH * HD, HD, 0, 0, None, 0, P(p1))
    R.ref_attn_decode(pos, n_act, M, max_len, P(q), P(k), P(v), P(p2))
    for m in range(n_act):
        nb = (pos + m) // 64 + 1
        assert np.array_equal(bits(p1[:, :nb, m]), bits(p2[:, :nb, m]))
    o1 = np.zeros((M, QH * HD), np.uint16); o2 = np.zeros_like(o1)
    L().orc_attn_reduce_v2(BF, C.byref(sh), pos, n_act, M, tgt, P(p2), P(gate), P(o1))
    R.ref_attn_reduce(pos, n_act, M, max_len, P(p2), P(gate), P(o2))
    assert np.array_equal(o1[:n_act], o2[:n_act])


def test_kv8_bitwise():
    rng = np.random.default_rng(1)
    for r in range(64):
        x = O.bf16_bits_to_f32(O.f32_to_bf16_bits((rng.standard_normal(256) * 10.0 ** rng.integers(-6, 3)).astype(np.float32)))
        x = np.ascontiguousarray(x)
        y1 = np.zeros(256, np.float32); y2 = np.zeros(256, np.float32)
        L().orc_kv8_rotate256(P(x), P(y1)); R.ref_kv8_rotate(P(x), P(y2))
        assert np.array_equal(bits(y1), bits(y2))
        L().orc_kv8_unrotate256(P(x), P(y1)); R.ref_kv8_unrotate(P(x), P(y2))
        assert np.array_equal(bits(y1), bits(y2))
        q1 = np.zeros(256, np.int8); q2 = np.zeros(256, np.int8)
        assert L().orc_kv8_encode256(P(x), P(q1)) == R.ref_kv8_encode(P(x), P(q2))
        assert np.array_equal(q1, q2)


def _kv8_prep_case(pos, n_act, M, max_len, seed):
    sh = _qwen_shape()
    rng = np.random.default_rng(seed)
    part = np.ascontiguousarray(rng.standard_normal((2, M, sh.qkv_n)).astype(np.float32))
    fa_small = np.ascontiguousarray((1 + 0.05 * rng.standard_normal(512)).astype(np.float32))
    rope = O.rope_table(1e7, ROT, max_len)
    return sh, part, fa_small, rope


@pytest.mark.parametrize("pos,n_act,paged", [(41, 2, False), (0, 1, False), (100, 3, True)])
def test_attn_prep_kv8_bitwise(pos, n_act, paged):
    """orc_attn_prep_kv8 (bf16, Qwen3.8's shape) against kv8_ref::prep: q rotated, K/V int8
    and scales bit for bit; a page table moves only the rows."""
    M, max_len = 3, 256
    sh, part, fa_small, rope = _kv8_prep_case(pos, n_act, M, max_len, 30 + pos)
    rng = np.random.default_rng(pos)
    k0 = rng.integers(-127, 128, (max_len, KVH, HD), dtype=np.int8)
    v0 = rng.integers(-127, 128, (max_len, KVH, HD), dtype=np.int8)
    ks0 = rng.integers(0, 0x3C00, (max_len, KVH), dtype=np.uint16)
    vs0 = rng.integers(0, 0x3C00, (max_len, KVH), dtype=np.uint16)
    pages = rng.permutation(max_len // 64).astype(np.uint32) if paged else None
    aq1 = np.zeros((M, QH, HD), np.float32); aq2 = np.zeros_like(aq1)
    g1 = np.zeros_like(aq1); g2 = np.zeros_like(aq1)
    rows = np.arange(max_len)
    if paged:  # logical position p of the reference's contiguous cache sits at the paged row
        rows = pages[rows // 64] * 64 + rows % 64
    k1, v1, ks1, vs1 = (np.empty_like(a) for a in (k0, v0, ks0, vs0))
    k1[rows], v1[rows], ks1[rows], vs1[rows] = k0, v0, ks0, vs0
    k2, v2, ks2, vs2 = k0.copy(), v0.copy(), ks0.copy(), vs0.copy()
    L().orc_attn_prep_kv8(BF, C.byref(sh), pos, n_act, M, P(part), 2, P(fa_small), P(fa_small[256:].copy()),
                          P(rope), P(aq1), P(g1), P(k1), P(v1), P(ks1), P(vs1), KVH * HD, HD, KVH, 1,
                          P(pages) if paged else None, 64 if paged else 0)
    R.ref_kv8_prep(pos, n_act, M, P(part), P(fa_small), P(rope), max_len, P(aq2), P(g2), P(k2), P(v2), P(ks2),
                   P(vs2))
    assert np.array_equal(bits(aq1[:n_act]), bits(aq2[:n_act]))
    assert np.array_equal(bits(g1[:n_act]), bits(g2[:n_act]))
    assert np.array_equal(k1[rows], k2) and np.array_equal(v1[rows], v2)
    assert np.array_equal(ks1[rows], ks2) and np.array_equal(vs1[rows], vs2)
    written = np.arange(pos, pos + n_act)
    assert not np.array_equal(k2[written], k0[written])  # the rows were rewritten


def test_attn_reduce_kv8_vs_reference_fp64_reader():
    """The rotated pair (orc_attn_decode_v2 on the int8 cache + orc_attn_reduce_v2_kv8)
    against kv8_ref::attend's fp64 reader with its fp64 un-rotation and the gated chain:
    cosine >= 0.99999 and within 2e-3 relative per head (the reference's reader bar)."""
    sh = _qwen_shape()
    M, max_len, pos, n_act = 1, 512, 300, 1
    tgt = 8
    rng = np.random.default_rng(5)
    q = np.ascontiguousarray(rng.standard_normal((M, QH, HD)).astype(np.float32))
    k = np.zeros((max_len, KVH, HD), np.int8); v = np.zeros_like(k)
    ks = np.zeros((max_len, KVH), np.uint16); vs = np.zeros_like(ks)
    for p in range(pos + 1):
        for j in range(KVH):
            x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.standard_normal(HD).astype(np.float32)))
            ks[p, j] = L().orc_kv8_encode256(P(np.ascontiguousarray(x)), P(k[p, j]))
            x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.standard_normal(HD).astype(np.float32)))
            vs[p, j] = L().orc_kv8_encode256(P(np.ascontiguousarray(x)), P(v[p, j]))
    gate = np.ascontiguousarray(rng.standard_normal((M, QH, HD)).astype(np.float32))
    part = np.zeros((QH, tgt, M, HD + 2), np.float32)
    L().orc_attn_decode_v2(BF, C.byref(sh), pos, n_act, M, tgt, P(q), 1, P(k), P(v), P(ks), P(vs),
                           KVH * HD, HD, KVH, 1, None, 0, P(part))
    out = np.zeros((M, QH * HD), np.uint16)
    L().orc_attn_reduce_v2_kv8(BF, C.byref(sh), pos, n_act, M, tgt, P(part), P(gate), P(out))
    got = O.bf16_bits_to_f32(out[0]).astype(np.float64).reshape(QH, HD)
    rot = np.zeros((QH, HD))
    L().orc_attn_reduce_v2(BF, C.byref(sh), pos, n_act, M, tgt, P(part), P(gate), P(out))
    rot[:] = O.bf16_bits_to_f32(out[0]).reshape(QH, HD)  # the same merge, left rotated
    o = np.zeros(HD); orot = np.zeros(HD)
    for h in range(QH):
        R.ref_kv8_attend(P(np.ascontiguousarray(q[0, h])), max_len, P(k), P(v), P(ks), P(vs), h // (QH // KVH),
                         pos + 1, P(o), P(orot))
        ob = O.bf16_bits_to_f32(O.f32_to_bf16_bits(o.astype(np.float32)))
        sg = np.float32(1) / (np.float32(1) + np.exp(-gate[0, h]))
        want = O.bf16_bits_to_f32(O.f32_to_bf16_bits((ob * sg).astype(np.float32))).astype(np.float64)
        cos = got[h] @ want / np.sqrt((got[h] @ got[h]) * (want @ want))
        assert cos >= 0.99999, (h, cos)
        assert np.max(np.abs(got[h] - want)) <= 2e-3 * np.max(np.abs(want)) + 1e-6, h
        # without the un-rotation the same partials miss the answer by far
        assert np.max(np.abs(rot[h] - want)) > 0.1 * np.max(np.abs(want)), h


class RefRoute(C.Structure):
    _fields_ = O.MoeRoute._fields_


@pytest.mark.parametrize("E,K", [(16, 4), (256, 8), (64, 8)])
def test_moe_route_bitwise(E, K):
    rng = np.random.default_rng(E + K)
    for t in range(20):
        lg = np.zeros(E + 16, np.float32)
        lg[:E + 1] = rng.uniform(-3, 3, E + 1)
        if t % 3 == 0:  # planted exact ties
            lg[5] = lg[E - 1] = lg[1] = 4.0
        a = O.MoeRoute(); b = RefRoute()
        L().orc_moe_route_fn(BF, P(lg), E, K, C.byref(a))
        R.ref_moe_route(P(lg), E, K, 2048, 512, E + 16, C.byref(b))
        assert list(a.ids[:K]) == list(b.ids[:K])
        for f in ("w", "p"):
            assert np.array_equal(np.array(getattr(a, f)[:K], np.float32), np.array(getattr(b, f)[:K], np.float32))
        assert a.p9 == b.p9 and a.sg == b.sg


def test_moe_split_dot_silu_combine_block():
    E, K, Hd, I, RN = 16, 4, 256, 128, 32
    rng = np.random.default_rng(12)
    # per expert: gate||up interleave16 -> layout-1 tiles; down -> layout-1 tiles
    gu_t, dn_t = [], []
    for b in range(E + 1):
        gq, gs = _rand(Hd, I, 100 + 3 * b)
        uq, us = _rand(Hd, I, 101 + 3 * b)
        oq = np.zeros((Hd // 8, 2 * I), np.uint32); os_ = np.zeros((Hd // 64, 2 * I), np.uint16)
        L().orc_interleave16_l0(P(gq), P(gs), P(uq), P(us), Hd, I, P(oq), P(os_))
        t = np.zeros((2 * I // 16) * (Hd // 64) * 136, np.uint32)
        L().orc_repack_layout1(P(oq), P(os_), Hd, 2 * I, P(t))
        gu_t.append(t)
        dq, ds = _rand(I, Hd, 102 + 3 * b)
        t2 = np.zeros((Hd // 16) * (I // 64) * 136, np.uint32)
        L().orc_repack_layout1(P(dq), P(ds), I, Hd, P(t2))
        dn_t.append(t2)
    gu = np.ascontiguousarray(np.concatenate(gu_t)); dn = np.ascontiguousarray(np.concatenate(dn_t))
    x = O.f32_to_bf16_bits(rng.uniform(-0.08, 0.08, Hd).astype(np.float32))
    for ks in (1, 2, 4):
        for n in range(0, 2 * I, 7):
            a = L().orc_moe_split_dot(BF, 1, P(gu_t[3]), None, Hd, 2 * I, n, P(x), ks)
            b = R.ref_moe_split_dot(P(gu_t[3]), Hd, n, P(x), ks)
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)
    for g, u in rng.uniform(-6, 6, (200, 2)).astype(np.float32):
        assert L().orc_moe_silu_up(BF, float(g), float(u)) == R.ref_moe_silu_up(float(g), float(u))
    for t in range(4):
        lg = np.zeros(RN, np.float32)
        lg[:E + 1] = rng.uniform(-3, 3, E + 1)
        resid = O.f32_to_bf16_bits(rng.uniform(-3, 3, Hd).astype(np.float32))
        a = O.MoeRoute()
        L().orc_moe_route_fn(BF, P(lg), E, K, C.byref(a))
        r1, r2 = resid.copy(), resid.copy()
        L().orc_moe_block(BF, 1, E, K, Hd, I, C.byref(a), P(x), P(gu), None, gu_t[0].size, 0, P(dn), None,
                          dn_t[0].size, 0, 2, 1, None, P(r1))
        R.ref_moe_block(P(lg), E, K, Hd, I, RN, P(x), P(gu), P(dn), 2, 1, P(r2))
        assert np.array_equal(r1, r2)
        d = np.ascontiguousarray(rng.standard_normal(K + 1).astype(np.float32))
        b = RefRoute()
        C.memmove(C.byref(b), C.byref(a), C.sizeof(a))
        assert L().orc_moe_combine(BF, P(d), C.byref(a), K, int(resid[0])) == \
            R.ref_moe_combine(P(d), C.byref(b), E, K, int(resid[0]))


def test_f16w_tile_layout_matches_reference_repack():
    K, N = 256, 48
    w = np.random.default_rng(3).integers(0, 65536, size=(N, K), dtype=np.uint32).astype(np.uint16)
    a = np.empty(K * N, np.uint16)
    b = np.empty(K * N, np.uint16)
    O.lib().orc_f16w_tile(O._p(w), K, N, O._p(a))
    R.ref_repack_bf16_tiled(O._p(w), K, N, O._p(b))
    assert np.array_equal(a, b)


def _moe_blocks(E, Hd, I, seed):
    """E + 1 experts' layout-1 gate||up (interleave16) and down blocks from the reference's
    random int4 weights"""
    gu_t, dn_t = [], []
    for b in range(E + 1):
        gq, gs = _rand(Hd, I, seed + 3 * b)
        uq, us = _rand(Hd, I, seed + 1 + 3 * b)
        oq = np.zeros((Hd // 8, 2 * I), np.uint32); os_ = np.zeros((Hd // 64, 2 * I), np.uint16)
        L().orc_interleave16_l0(P(gq), P(gs), P(uq), P(us), Hd, I, P(oq), P(os_))
        t = np.zeros((2 * I // 16) * (Hd // 64) * 136, np.uint32)
        L().orc_repack_layout1(P(oq), P(os_), Hd, 2 * I, P(t))
        gu_t.append(t)
        dq, ds = _rand(I, Hd, seed + 2 + 3 * b)
        t2 = np.zeros((Hd // 16) * (I // 64) * 136, np.uint32)
        L().orc_repack_layout1(P(dq), P(ds), I, Hd, P(t2))
        dn_t.append(t2)
    return np.ascontiguousarray(np.concatenate(gu_t)), np.ascontiguousarray(np.concatenate(dn_t))


@pytest.mark.parametrize("E,K,T", [(16, 4, 37), (32, 8, 21)])
def test_moe_prefill_bitwise_pf_moe_ref(E, K, T):
    """orc_moe_prefill (token by token) against pf_moe_ref's sort + dequant_block + gemm_rows +
    silu_row + grouped walk + combine_token (bf16): every residual bit, with routes that send
    several tokens to the same experts."""
    Hd, I = 512, 128
    gu, dn = _moe_blocks(E, Hd, I, 300 + E)
    rng = np.random.default_rng(E + T)
    route = np.zeros((T, 32), np.uint32)
    for t in range(T):
        lg = np.zeros(E + 16, np.float32)
        lg[:E + 1] = rng.uniform(-3, 3, E + 1)
        if t % 4 == 0:
            lg[:E] = lg[:E] * 0.05  # near-uniform: many tokens share experts
        r = O.MoeRoute()
        L().orc_moe_route_fn(BF, P(lg), E, K, C.byref(r))
        route[t, :K] = list(r.ids[:K])
        route[t, 8:8 + K] = np.array(r.w[:K], np.float32).view(np.uint32)
        route[t, 16] = np.float32(r.sg).view(np.uint32)
    x = O.f32_to_bf16_bits(rng.uniform(-0.5, 0.5, (T, Hd)).astype(np.float32))
    resid = O.f32_to_bf16_bits(rng.uniform(-3, 3, (T, Hd)).astype(np.float32))
    a, b = resid.copy(), resid.copy()
    L().orc_moe_prefill(BF, E, K, Hd, I, P(route), P(x), P(gu), P(dn), P(a), T)
    R.ref_pf_moe_block(P(route), T, P(x), P(gu), P(dn), E, K, Hd, I, P(b))
    assert np.array_equal(a, b)
    assert not np.array_equal(a, resid)


def _int8_rows(N, K, seed):
    """bf16 rows N(0, 0.02) with lm_head_int8_test's special rows: one all zero, one with a
    large positive outlier, one whose largest magnitude is negative."""
    rng = np.random.default_rng(seed)
    w = O.f32_to_bf16_bits((0.02 * rng.standard_normal((N, K))).astype(np.float32))
    w[5] = 0
    w[3, 17] = O.f32_to_bf16_bits(np.float32(0.9))
    w[7, K - 1] = O.f32_to_bf16_bits(np.float32(-1.5))
    return w


@pytest.mark.parametrize("N,K,seed", [(64, 256, 1234), (48, 5120, 7)])
def test_int8_head_quantiser_bitwise_lm_head_int8(N, K, seed):
    """orc_quantise_row_int8 against the reference's quantise_int8_tiled (lm_head_int8.cc,
    compiled into _ref): every scale's bits and every q at int8_tiled_index."""
    w = _int8_rows(N, K, seed)
    qt = np.zeros(N * K, np.int8)
    st = np.zeros(N, np.float32)
    R.ref_quantise_int8_tiled(P(w), K, N, P(qt), P(st))
    wf = O.bf16_bits_to_f32(w).astype(np.float32)
    for n in range(N):
        q = np.zeros(K, np.int8)
        s = L().orc_quantise_row_int8(P(np.ascontiguousarray(wf[n])), K, P(q))
        assert np.float32(s).view(np.uint32) == st[n].view(np.uint32), n
        idx = np.array([R.ref_int8_tiled_index(K, k, n) for k in range(K)])
        assert np.array_equal(qt[idx], q), n
    assert st[5] == 0 and not np.any(qt[[R.ref_int8_tiled_index(K, k, 5) for k in range(K)]])


def _rtn_rows(N, K, seed):
    """bf16 [N][K] with the quantiser's corner cases: an all-zero group, a group whose largest
    magnitude makes w / s land on .5 ties, subnormal-scale groups, negative extremes"""
    rng = np.random.default_rng(seed)
    w = O.f32_to_bf16_bits((0.05 * rng.standard_normal((N, K))).astype(np.float32))
    w[3, 64:128] = 0
    # amax 7.5 -> s = 1.0 exactly: the row is k/2 steps, every odd k a tie (round to even)
    w[4, :64] = O.f32_to_bf16_bits(np.arange(-64, 64, 2, dtype=np.float32)[:64] * 0.125 - 0.0)
    w[4, 0] = O.f32_to_bf16_bits(np.float32([7.5]))[0]
    w[5, 128:192] = O.f32_to_bf16_bits(rng.uniform(-1e-6, 1e-6, 64).astype(np.float32))  # s16 subnormal
    w[6, 192:256] = O.f32_to_bf16_bits(-np.abs(rng.standard_normal(64)).astype(np.float32))
    return np.ascontiguousarray(w)


@pytest.mark.parametrize("N,K,seed", [(32, 256, 3), (16, 1024, 11)])
def test_rtn_int4_quantiser_bitwise_rtn_h(N, K, seed):
    """orc_rtn_int4_g64 against the reference's rtn_int4_g64 (src/loader/rtn.h, compiled into
    _ref): every qweight word and every scale, bit for bit, corner cases included."""
    w = _rtn_rows(N, K, seed)
    q1 = np.zeros((K // 8, N), np.uint32); s1 = np.zeros((K // 64, N), np.uint16)
    q2 = np.zeros_like(q1); s2 = np.zeros_like(s1)
    L().orc_rtn_int4_g64(P(w), K, N, P(q1), P(s1))
    R.ref_rtn_int4_g64(P(w), K, N, P(q2), P(s2))
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    assert s1[1, 3] == 0 and np.all(q1[8:16, 3] == 0x88888888)  # the zero group: s 0, q 8
