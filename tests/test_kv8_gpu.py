"""The int8 KV cache end to end on the GPU: the writer (attn_prep_kv8, kv8.cl:287-408) and the
rotated reader pair (attn_decode_v2_kv8 + attn_reduce_v2_kv8, kv8.cl:535, :814) through the
C ABI against the CPU oracle.

Bars (kv8_kernels_test / kv8_ref.h:1-12): the writer bitwise the oracle (q rotated, K/V int8
and fp16 scales; every op of the chain is one fp32 rounding in a fixed order), zero and
subnormal-scale rows included; the reader's output within rel 2e-3 and cosine >= 0.99999 of
the fp64 attention over the same int8 cache with an fp64 un-rotation; the reduce's
un-rotation within 2 fp16 ulp of the oracle's on the device's own partials."""
import ctypes as C

import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16
L = O.lib
HD = 256
SIGN_WORDS = [0xA197D809, 0xA6850592, 0xB205A73E, 0x20AFA769, 0x45C2CF64, 0xBEAEAACB, 0x75F39ADD, 0x2385A70C]
SIGNS = np.array([-1.0 if (SIGN_WORDS[j >> 5] >> (j & 31)) & 1 else 1.0 for j in range(HD)])
H256 = hadamard(HD).astype(np.float64)


def unrotate64(y):
    """R^T in fp64 along the last axis: FWHT(s * y) / 16."""
    return (y * SIGNS) @ H256 / 16.0


def ctrl_dev(pos, n_act):
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos, n_act
    return dev(c)


def prep_inputs(sh, M, S, Lm, seed):
    rng = np.random.default_rng(seed)
    part = rng.standard_normal((S, M, sh.qkv_n)).astype(np.float32)
    qn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32)
    rope = O.rope_table(1e6, sh.rot_dim, Lm)
    return part, qn, kn, rope


def gpu_prep_kv8(sh, part, S, M, pos, n_act, qn, kn, rope, k8, v8, ks, vs, pages=None, page=0):
    QH = sh.q_heads
    Lm = k8.shape[1]
    print(f"attn_prep_kv8 QH={QH} KVH={sh.kv_heads} pos={pos} M={M} n_act={n_act} paged={pages is not None}",
          flush=True)
    ctrl = ctrl_dev(pos, n_act)
    dq = empty((M, QH, HD), np.float32)
    dg = empty((M, QH, HD), np.float32)
    dq.zero_(); dg.zero_()
    dk, dv, dks, dvs = dev(k8), dev(v8), dev(ks), dev(vs)
    keep = [dev(part), dev(qn), dev(kn), dev(rope), dev(pages)]
    mi.call("mi_attn_prep_kv8", ptr(ctrl), ptr(keep[0]), S, M, mi.shape_ref(sh), ptr(keep[1]), ptr(keep[2]),
            ptr(keep[3]), ptr(dq), ptr(dg), ptr(dk), ptr(dv), ptr(dks), ptr(dvs), HD, Lm * HD, 1, Lm,
            ptr(keep[4]), page, Lm, stream())
    sync()
    return (host(dq, np.float32), host(dg, np.float32), host(dk, np.int8), host(dv, np.int8),
            host(dks, np.uint16), host(dvs, np.uint16))


def oracle_prep_kv8(sh, part, S, M, pos, n_act, qn, kn, rope, k8, v8, ks, vs, pages=None, page=0):
    Lm = k8.shape[1]
    aq = np.zeros((M, sh.q_heads, HD), np.float32)
    ag = np.zeros_like(aq)
    k2, v2, ks2, vs2 = k8.copy(), v8.copy(), ks.copy(), vs.copy()
    L().orc_attn_prep_kv8(F16, C.byref(sh), pos, n_act, M, O._p(part), S, O._p(qn), O._p(kn), O._p(rope),
                          O._p(aq), O._p(ag), O._p(k2), O._p(v2), O._p(ks2), O._p(vs2), HD, Lm * HD, 1, Lm,
                          O._p(pages), page)
    return aq, ag, k2, v2, ks2, vs2


@pytest.mark.parametrize("shape,paged", [("qwen38", False), ("qwen38", True), ("cfg4", False)])
def test_attn_prep_kv8_bitwise(shape, paged):
    if shape == "qwen38":
        sh = O.attn_shape(24, 4, HD, rot_dim=64, gated=True)
    else:
        sh = O.attn_shape(16, 2, HD)
    M, n_act, pos, S, Lm = 3, 3, 700, 2, 1024
    part, qn, kn, rope = prep_inputs(sh, M, S, Lm, 11 + paged)
    KVH = sh.kv_heads
    # row 0: kv head 0's K and V all zero (scale 0, every q 0); kv head 1's V tiny, so its
    # scale is an f16 subnormal
    part[:, 0, sh.k_off:sh.k_off + HD] = 0.0
    part[:, 0, sh.v_off:sh.v_off + HD] = 0.0
    part[:, 0, sh.v_off + HD:sh.v_off + 2 * HD] *= 3e-5
    rng = np.random.default_rng(2)
    k8 = rng.integers(-127, 128, (KVH, Lm, HD), dtype=np.int8)
    v8 = rng.integers(-127, 128, (KVH, Lm, HD), dtype=np.int8)
    ks = rng.integers(0, 0x3C00, (KVH, Lm), dtype=np.uint16)
    vs = rng.integers(0, 0x3C00, (KVH, Lm), dtype=np.uint16)
    pages = rng.permutation(Lm // 64).astype(np.uint32) if paged else None
    page = 64 if paged else 0
    got = gpu_prep_kv8(sh, part, S, M, pos, n_act, qn, kn, rope, k8, v8, ks, vs, pages, page)
    want = oracle_prep_kv8(sh, part, S, M, pos, n_act, qn, kn, rope, k8, v8, ks, vs, pages, page)
    names = ["attn_q", "attn_gate", "k8", "v8", "k_scale", "v_scale"]
    for name, g, w in zip(names, got, want):
        if name == "attn_gate" and not sh.gated:
            continue
        gv = g.view(np.uint32) if g.dtype == np.float32 else g
        wv = w.view(np.uint32) if w.dtype == np.float32 else w
        assert np.array_equal(gv, wv), name
    row0 = pages[pos // 64] * 64 + pos % 64 if paged else pos
    assert want[4][0, row0] == 0 and not want[2][0, row0].any()            # the all-zero row
    assert 0 < want[5][1, row0] < 0x0400                                     # subnormal scale


def quantised_cache(KVH, n, Lm, seed):
    """An int8 cache whose rows [0, n) are the writer's encoding of fp16 N(0, 1) rows."""
    rng = np.random.default_rng(seed)
    k8 = np.zeros((KVH, Lm, HD), np.int8); v8 = np.zeros_like(k8)
    ks = np.zeros((KVH, Lm), np.uint16); vs = np.zeros_like(ks)
    for j in range(KVH):
        for p in range(n):
            x = O.f16_bits_to_f32(O.f32_to_f16_bits(rng.standard_normal(HD).astype(np.float32)))
            ks[j, p] = L().orc_kv8_encode256(O._p(np.ascontiguousarray(x)), O._p(k8[j, p]))
            x = O.f16_bits_to_f32(O.f32_to_f16_bits(rng.standard_normal(HD).astype(np.float32)))
            vs[j, p] = L().orc_kv8_encode256(O._p(np.ascontiguousarray(x)), O._p(v8[j, p]))
    return k8, v8, ks, vs


@pytest.mark.parametrize("QH,KVH,gated", [(16, 2, False), (24, 4, True)])
def test_writer_then_rotated_reader_vs_fp64(QH, KVH, gated):
    """One decode step on the int8 path: attn_prep_kv8 writes position pos, attn_decode
    (int8) and attn_reduce_kv8 read positions [0, pos]. Against the fp64 attention over the
    same int8 cache with an fp64 un-rotation (kv8_ref::attend's bar), and the oracle pair."""
    sh = O.attn_shape(QH, KVH, HD, rot_dim=64 if gated else None, gated=gated)
    M, S, Lm, tgt, pos = 1, 2, 1024, 16, 900
    part, qn, kn, rope = prep_inputs(sh, M, S, Lm, 21)
    k8, v8, ks, vs = quantised_cache(KVH, pos, Lm, 22)
    aq, ag, k8, v8, ks, vs = gpu_prep_kv8(sh, part, S, M, pos, 1, qn, kn, rope, k8, v8, ks, vs)
    ctrl = ctrl_dev(pos, 1)
    dq, dg = dev(aq), dev(ag)
    dk, dv, dks, dvs = dev(k8), dev(v8), dev(ks), dev(vs)
    dpart = empty((QH, tgt, M, HD + 2), np.float32)
    out = empty((M, QH * HD), np.uint16)
    print(f"kv8 reader QH={QH} KVH={KVH} gated={gated} pos={pos}", flush=True)
    mi.call("mi_attn_decode", ptr(ctrl), ptr(dq), 1, ptr(dk), ptr(dv), ptr(dks), ptr(dvs), HD, Lm * HD, 1, Lm,
            None, 0, Lm, ptr(dpart), M, tgt, mi.shape_ref(sh), stream())
    mi.call("mi_attn_reduce_kv8", ptr(ctrl), ptr(dpart), ptr(dg) if gated else None, ptr(out), M, tgt, Lm,
            mi.shape_ref(sh), stream())
    sync()
    got = O.f16_bits_to_f32(host(out, np.uint16)[0]).astype(np.float64).reshape(QH, HD)
    G = QH // KVH
    o_rot = np.zeros((QH, HD))
    for h in range(QH):
        L().orc_attend64(C.byref(sh), O._p(np.ascontiguousarray(aq[0, h])), h // G, pos + 1, 1, F16, O._p(k8),
                         O._p(v8), O._p(ks), O._p(vs), HD, Lm * HD, 1, Lm, None, 0, O._p(o_rot[h]))
    o = unrotate64(o_rot)
    if gated:
        ob = O.f16_bits_to_f32(O.f32_to_f16_bits(o.astype(np.float32))).astype(np.float64)
        want = ob / (1.0 + np.exp(-ag[0].astype(np.float64)))
    else:
        want = o
    err = np.abs(got - want)
    assert np.all(err <= 2e-3 * np.abs(want) + 2e-3 * np.abs(want).max(axis=-1, keepdims=True)), err.max()
    cos = (got * want).sum(-1) / np.sqrt((got * got).sum(-1) * (want * want).sum(-1))
    assert cos.min() >= 0.99999
    # the oracle's own pair on the device's partials: within 2 fp16 ulp
    ref = np.zeros((M, QH * HD), np.uint16)
    L().orc_attn_reduce_v2_kv8(F16, C.byref(sh), pos, 1, M, tgt, O._p(host(dpart, np.float32).copy()),
                               O._p(ag) if gated else None, O._p(ref))
    a = O.f16_bits_to_f32(host(out, np.uint16)).astype(np.float64)
    b = O.f16_bits_to_f32(ref).astype(np.float64)
    assert np.all(np.abs(a - b) <= np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10 * 2.01)


def test_reduce_kv8_is_reduce_then_unrotation():
    """attn_reduce_kv8 on arbitrary partials equals the plain reduce's merge followed by the
    un-rotation: checked against the oracle's kv8 reduce within 2 fp16 ulp, and the plain
    reduce's output (left rotated) is far from it."""
    QH, KVH, tgt, pos = 8, 2, 8, 1000
    sh = O.attn_shape(QH, KVH, HD)
    rng = np.random.default_rng(7)
    part = rng.standard_normal((QH, tgt, 1, HD + 2)).astype(np.float32)
    part[..., 1] = np.abs(part[..., 1]) + 1.0  # block sums are positive
    ctrl = ctrl_dev(pos, 1)
    dp = dev(part)
    out = empty((1, QH * HD), np.uint16)
    plain = empty((1, QH * HD), np.uint16)
    mi.call("mi_attn_reduce_kv8", ptr(ctrl), ptr(dp), None, ptr(out), 1, tgt, 0, mi.shape_ref(sh), stream())
    mi.call("mi_attn_reduce", ptr(ctrl), ptr(dp), None, ptr(plain), 1, tgt, 0, mi.shape_ref(sh), stream())
    sync()
    ref = np.zeros((1, QH * HD), np.uint16)
    L().orc_attn_reduce_v2_kv8(F16, C.byref(sh), pos, 1, 1, tgt, O._p(part), None, O._p(ref))
    a = O.f16_bits_to_f32(host(out, np.uint16)).astype(np.float64)
    b = O.f16_bits_to_f32(ref).astype(np.float64)
    assert np.all(np.abs(a - b) <= np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10 * 2.01)
    p = O.f16_bits_to_f32(host(plain, np.uint16)).astype(np.float64).reshape(QH, HD)
    assert np.allclose(unrotate64(p), b.reshape(QH, HD), rtol=0, atol=4e-3 * np.abs(b).max())
    assert np.abs(p - b.reshape(QH, HD)).max() > 0.1 * np.abs(b).max()
