"""The many-row verify attention (mi_attn_verify, the role of attn_verify_dpas at 16 q / 2 kv
heads, attn_verify_dpas.cl:383, bound by verify_attn.h:93-96) vs the fp64 attention of the
oracle, at M = 16, 32, 64 rows.

Bars: each (row, head) within rel 2e-3 of the fp64 reference and cosine >= 0.99999 (the
reference holds its verify attention to fp64 by cosine: attn_verify_dpas.cl's PSPLIT note);
property R (a row bitwise equal at the same key count in any M launch, attn_verify_dpas.cl's
"Property R" section) across M = 16, 32, 64 and across row lists that cross a block-stride
change; a paged cache bitwise the contiguous one; the bind rule of verify_attn.h:93-100."""
import ctypes as C

import numpy as np
import pytest

from mipkg import dev, empty, host, mi, ptr, stream, sync
from test_attn_gpu import check_close, ctrl_dev, fp64_attention, make_kv

pytestmark = pytest.mark.gpu
QH, KVH = 16, 2


def shape(HD):
    return mi.AttnShape(QH, KVH, HD, HD, 0, (QH + 2 * KVH) * HD, QH * HD, (QH + KVH) * HD,
                        float(np.float32(1 / np.sqrt(HD))), 1e-6)


def verify(sh, q, k, v, pos, M, tgt, pages=None, page=0):
    HD = sh.head_dim
    Lm = k.shape[1]
    print(f"attn_verify HD={HD} pos={pos} M={M} tgt={tgt} paged={pages is not None}", flush=True)
    ctrl = ctrl_dev(pos, M)
    part = empty((QH, tgt, M, HD + 2), np.float32)
    out = empty((M, QH * HD), np.uint16)
    dk, dv, dq, dpg = dev(k), dev(v), dev(q), dev(pages)
    shp = mi.shape_ref(sh)
    mi.call("mi_attn_verify", ptr(ctrl), ptr(dq), ptr(dk), ptr(dv), HD, Lm * HD, ptr(dpg), page, Lm, ptr(part), M,
            tgt, shp, stream())
    mi.call("mi_attn_reduce", ptr(ctrl), ptr(part), None, ptr(out), M, tgt, Lm, shp, stream())
    sync()
    return host(out, np.uint16)


@pytest.mark.parametrize("HD,pos,tgt", [(256, 1000, 64), (256, 4083, 32), (128, 2040, 32)])
def test_verify_rows_vs_fp64_and_property_r(HD, pos, tgt):
    # (256, 4083, 32) and (128, 2040, 32): the rows' key counts cross a stride change of the
    # block walk (ppw(L) at tgt 32 grows from 64 to 128 past L = 2048, and to 192 past 4096)
    Lm = pos + 64 + 16
    sh = shape(HD)
    k, v, _, _ = make_kv(0, KVH, Lm, HD, 7 + pos)
    rng = np.random.default_rng(pos)
    q = rng.standard_normal((64, QH, HD)).astype(np.float32)
    outs = {}
    for M in (16, 32, 64):
        outs[M] = verify(sh, q[:M].copy(), k, v, pos, M, tgt)
    for M in (32, 64):  # property R: rows 0..15 (0..31) bitwise the smaller list's
        np.testing.assert_array_equal(outs[M][:16], outs[16])
    np.testing.assert_array_equal(outs[64][:32], outs[32])
    for m in (0, 7, 15, 16, 31, 40, 63):
        want = fp64_attention(sh, q[m], 0, k, v, None, None, pos + m + 1)
        check_close(outs[64][m:m + 1], want.reshape(1, -1))


def test_verify_paged_is_contiguous():
    HD, pos, tgt, P = 256, 3000, 64, 64
    Lm = 4096
    sh = shape(HD)
    k, v, _, _ = make_kv(0, KVH, Lm, HD, 3)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((16, QH, HD)).astype(np.float32)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    # the paged cache: logical position p at row pages[p / P] * P + p % P
    kp, vp = np.empty_like(k), np.empty_like(v)
    for lp in range(Lm // P):
        kp[:, pages[lp] * P:(pages[lp] + 1) * P] = k[:, lp * P:(lp + 1) * P]
        vp[:, pages[lp] * P:(pages[lp] + 1) * P] = v[:, lp * P:(lp + 1) * P]
    a = verify(sh, q, k, v, pos, 16, tgt)
    b = verify(sh, q, kp, vp, pos, 16, tgt, pages, P)
    np.testing.assert_array_equal(b, a)


def test_verify_partial_rows_and_replay():
    """n_act < M: only the live rows are written; a second launch gives the same bits."""
    HD, pos, tgt = 256, 500, 64
    Lm = 1024
    sh = shape(HD)
    k, v, _, _ = make_kv(0, KVH, Lm, HD, 9)
    q = np.random.default_rng(1).standard_normal((32, QH, HD)).astype(np.float32)
    ctrl = ctrl_dev(pos, 20)
    part = empty((QH, tgt, 32, HD + 2), np.float32)
    out = dev(np.full((32, QH * HD), 0x7E00, np.uint16))
    dk, dv, dq = dev(k), dev(v), dev(q)
    shp = mi.shape_ref(sh)
    res = []
    for _ in range(2):
        mi.call("mi_attn_verify", ptr(ctrl), ptr(dq), ptr(dk), ptr(dv), HD, Lm * HD, None, 0, Lm, ptr(part), 32, tgt,
                shp, stream())
        mi.call("mi_attn_reduce", ptr(ctrl), ptr(part), None, ptr(out), 32, tgt, Lm, shp, stream())
        sync()
        res.append(host(out, np.uint16).copy())
    np.testing.assert_array_equal(res[1], res[0])
    assert np.all(res[0][20:] == 0x7E00)
    full = verify(sh, q, k, v, pos, 32, tgt)
    np.testing.assert_array_equal(res[0][:20], full[:20])
