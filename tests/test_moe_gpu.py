"""Mixture-of-experts block on the GPU (router GEMV, routing, expert gate||up, down + combine)
through the C ABI against the CPU oracle (the restated tests/kernels/moe_ref.h twins).

Bars (moe_ref_test / moe_test): the router GEMV bitwise the oracle's gemv_bf16 order; expert
ids bit-exact (ties to the lower id) and w_k / s exact or 1 fp16 ulp (exp); the gate||up
output within 2 fp16 ulp (the SiLU's exp) and mostly bitwise; the down + combine bitwise the
oracle's on the same h (no exp on that path); the whole block's residual within 2 fp16 ulp of
the oracle's. Config 4's shape: hidden 2048, 256 experts, top 8 + shared, expert inter 512."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16
ROUTE_WORDS = 32


def layout1_blocks(n_blocks, K, N, rng):
    """n_blocks int4 g64 layout-1 weight blocks of K x N: per (n_tile, k_group) 128 u32 of
    nibbles [8 k-octets][16 n] then 16 f16 scales U(0.002, 0.02)."""
    tiles = n_blocks * (N // 16) * (K // 64)
    w = rng.integers(0, 2**32, size=(tiles, 136), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, (tiles, 16)).astype(np.float32))
    w[:, 128:] = sc.view(np.uint32).reshape(tiles, 8)
    return w.reshape(-1)


class Moe:
    def __init__(self, seed, E=256, top_k=8, hidden=2048, inter=512, router_n=272):
        rng = np.random.default_rng(seed)
        self.E, self.top_k, self.hidden, self.inter, self.router_n = E, top_k, hidden, inter, router_n
        w = np.zeros((router_n, hidden), np.float32)
        w[:E + 1] = 0.02 * rng.standard_normal((E + 1, hidden))
        self.router_rm = O.f32_to_f16_bits(w)
        self.router = np.empty(router_n * hidden, np.uint16)
        O.lib().orc_f16w_tile(O._p(self.router_rm), hidden, router_n, O._p(self.router))
        self.gu = layout1_blocks(E + 1, hidden, 2 * inter, rng)
        self.dn = layout1_blocks(E + 1, inter, hidden, rng)
        self.gu_block = (2 * inter // 16) * (hidden // 64) * 136
        self.dn_block = (hidden // 16) * (inter // 64) * 136
        self.d_router, self.d_gu, self.d_dn = dev(self.router), dev(self.gu), dev(self.dn)

    def oracle_logits(self, x, M, ksplit=16):
        out = np.empty((M, self.router_n), np.float32)
        O.lib().orc_gemv_f16w(F16, O._p(self.router), O._p(x), M, self.hidden, self.router_n, ksplit, O._p(out))
        return out

    def oracle_route(self, logits_row):
        r = O.MoeRoute()
        O.lib().orc_moe_route_fn(F16, O._p(np.ascontiguousarray(logits_row, np.float32)), self.E, self.top_k,
                                 C.byref(r))
        return r


def route_struct_from_row(row, top_k):
    r = O.MoeRoute()
    for k in range(top_k):
        r.ids[k] = int(row[k])
        r.w[k] = float(row[8 + k:9 + k].view(np.float32)[0])
        r.p[k] = float(row[17 + k:18 + k].view(np.float32)[0])
    r.p9 = float(row[25:26].view(np.float32)[0])
    r.sg = float(row[16:17].view(np.float32)[0])
    return r


def f16_ulps(a, b):
    """distance in fp16 ulps between fp16 bit patterns (same-sign values)"""
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(sa - sb)


def gpu_block(mo, x, M, resid):
    print(f"moe block E={mo.E} top_k={mo.top_k} hidden={mo.hidden} inter={mo.inter} M={M}", flush=True)
    dx = dev(x)
    logits = empty((M, mo.router_n), np.float32)
    route = empty((M, ROUTE_WORDS), np.uint32)
    h = empty((M, mo.top_k + 1, mo.inter), np.uint16)
    dres = dev(resid)
    mi.call("mi_gemv_f16w", ptr(mo.d_router), ptr(dx), ptr(logits), M, mo.hidden, mo.router_n, 16, stream())
    mi.call("mi_moe_route", ptr(logits), ptr(route), M, mo.E, mo.top_k, mo.router_n, stream())
    mi.call("mi_moe_gate_up", ptr(route), ptr(dx), ptr(mo.d_gu), ptr(h), M, mo.E, mo.top_k, mo.hidden, mo.inter,
            stream())
    mi.call("mi_moe_down", ptr(route), ptr(h), ptr(mo.d_dn), ptr(dres), M, mo.E, mo.top_k, mo.hidden, mo.inter,
            stream())
    sync()
    return (host(logits, np.float32), host(route, np.uint32), host(h, np.uint16), host(dres, np.uint16))


@pytest.fixture(scope="module")
def moe256():
    return Moe(1)


@pytest.mark.parametrize("M", [1, 3])
def test_router_gemv_bitwise(moe256, M):
    mo = moe256
    x = O.f32_to_f16_bits(np.random.default_rng(10 + M).standard_normal((M, mo.hidden)).astype(np.float32))
    for ksplit in (16, 4):
        dx = dev(x)
        out = empty((M, mo.router_n), np.float32)
        mi.call("mi_gemv_f16w", ptr(mo.d_router), ptr(dx), ptr(out), M, mo.hidden, mo.router_n, ksplit, stream())
        sync()
        got = host(out, np.float32)
        want = mo.oracle_logits(x, M, ksplit)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), ksplit


def test_route_vs_oracle_and_planted_ties():
    E, top_k, router_n = 64, 8, 80
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(router_n).astype(np.float32) for _ in range(3)]
    # exact ties: equal logits straddling the top-k boundary, and an all-equal row
    t = rng.standard_normal(router_n).astype(np.float32)
    t[[3, 9, 17, 40, 41, 60]] = 3.0
    t[[5, 7]] = 2.5
    rows.append(t)
    rows.append(np.full(router_n, 0.25, np.float32))
    lg = np.stack(rows)
    M = lg.shape[0]
    dl = dev(lg)
    route = empty((M, ROUTE_WORDS), np.uint32)
    mi.call("mi_moe_route", ptr(dl), ptr(route), M, E, top_k, router_n, stream())
    sync()
    got = host(route, np.uint32)
    for m in range(M):
        r = O.MoeRoute()
        O.lib().orc_moe_route_fn(F16, O._p(lg[m]), E, top_k, C.byref(r))
        assert list(got[m, :top_k]) == list(r.ids[:top_k]), m
        gw = got[m, 8:8 + top_k].view(np.float32)
        ww = np.array(r.w[:top_k], np.float32)
        assert np.all(f16_ulps(O.f32_to_f16_bits(gw), O.f32_to_f16_bits(ww)) <= 1), m
        gsg = got[m, 16:17].view(np.float32)
        assert f16_ulps(O.f32_to_f16_bits(gsg), O.f32_to_f16_bits(np.float32([r.sg])))[0] <= 1
    # all-equal row: ids 0..7 (ties go to the lower id), equal weights 1/8
    assert list(got[4, :top_k]) == list(range(8))
    assert np.all(got[4, 8:16].view(np.float32) == np.float32(0.125))


@pytest.mark.parametrize("M", [1, 2])
def test_gate_up_and_down_vs_oracle(moe256, M):
    mo = moe256
    rng = np.random.default_rng(20 + M)
    x = O.f32_to_f16_bits(rng.standard_normal((M, mo.hidden)).astype(np.float32))
    resid = O.f32_to_f16_bits(rng.standard_normal((M, mo.hidden)).astype(np.float32))
    logits, route, h, res_gpu = gpu_block(mo, x, M, resid)
    assert np.array_equal(logits.view(np.uint32), mo.oracle_logits(x, M).view(np.uint32))
    for m in range(M):
        r_or = mo.oracle_route(logits[m])
        assert list(route[m, :mo.top_k]) == list(r_or.ids[:mo.top_k])
        r = route_struct_from_row(route[m], mo.top_k)
        # gate||up: the oracle's whole block on the GPU's route gives its h
        h_or = np.empty((mo.top_k + 1, mo.inter), np.uint16)
        res_or = resid[m].copy()
        O.lib().orc_moe_block(F16, 1, mo.E, mo.top_k, mo.hidden, mo.inter, C.byref(r), O._p(x[m]), O._p(mo.gu),
                              None, mo.gu_block, 0, O._p(mo.dn), None, mo.dn_block, 0, 4, 2, O._p(h_or),
                              O._p(res_or))
        u = f16_ulps(h[m], h_or)
        assert u.max() <= 2 and np.mean(u == 0) >= 0.95, (u.max(), np.mean(u == 0))
        # down + combine on the GPU's own h: bitwise the oracle's split dots + combine
        cols = range(0, mo.hidden, 61)
        for n in cols:
            d = np.empty(mo.top_k + 1, np.float32)
            for slot in range(mo.top_k + 1):
                e = r.ids[slot] if slot < mo.top_k else mo.E
                blk = C.c_void_p(mo.dn.ctypes.data + 4 * e * mo.dn_block)
                d[slot] = O.lib().orc_moe_split_dot(F16, 1, blk, None, mo.inter, mo.hidden, n,
                                                    O._p(np.ascontiguousarray(h[m, slot])), 2)
            want = O.lib().orc_moe_combine(F16, O._p(d), C.byref(r), mo.top_k, int(resid[m, n]))
            assert int(res_gpu[m, n]) == int(want), n
        # the whole block: within 2 fp16 ulp of the oracle's (exp differences in the SiLU)
        assert f16_ulps(res_gpu[m], res_or).max() <= 2


@pytest.mark.parametrize("E,hidden,inter,M", [(256, 2048, 512, 1), (256, 2048, 512, 3), (16, 512, 128, 2)])
def test_routed_gate_up_is_route_then_gate_up(E, hidden, inter, M):
    """mi_moe_gate_up_routed (routing inside the gate||up launch) writes the route rows and h
    bitwise mi_moe_route + mi_moe_gate_up, including planted exact ties in the logits."""
    mo = Moe(3, E=E, hidden=hidden, inter=inter, router_n=E + 16)
    print(f"routed gate_up E={E} hidden={hidden} inter={inter} M={M}", flush=True)
    rng = np.random.default_rng(E + M)
    lg = rng.standard_normal((M, mo.router_n)).astype(np.float32)
    lg[0, [1, 5, 9, 13]] = 2.75  # a tie straddling the top-k boundary
    x = O.f32_to_f16_bits(rng.standard_normal((M, hidden)).astype(np.float32))
    dl, dx = dev(lg), dev(x)
    r1, r2 = empty((M, ROUTE_WORDS), np.uint32), empty((M, ROUTE_WORDS), np.uint32)
    h1 = empty((M, mo.top_k + 1, inter), np.uint16)
    h2 = empty((M, mo.top_k + 1, inter), np.uint16)
    mi.call("mi_moe_route", ptr(dl), ptr(r1), M, E, mo.top_k, mo.router_n, stream())
    mi.call("mi_moe_gate_up", ptr(r1), ptr(dx), ptr(mo.d_gu), ptr(h1), M, E, mo.top_k, hidden, inter, stream())
    mi.call("mi_moe_gate_up_routed", ptr(dl), mo.router_n, ptr(r2), ptr(dx), ptr(mo.d_gu), ptr(h2), M, E,
            mo.top_k, hidden, inter, stream())
    sync()
    assert np.array_equal(host(r1, np.uint32), host(r2, np.uint32))
    assert np.array_equal(host(h1, np.uint16), host(h2, np.uint16))


@pytest.mark.parametrize("E,hidden,inter,M", [(256, 2048, 512, 1), (256, 2048, 512, 3), (16, 4096, 128, 8),
                                              (16, 512, 128, 2)])
def test_down_norm_is_down_then_norm_rows(E, hidden, inter, M):
    """mi_moe_down_norm writes the residual of mi_moe_down and the x / rstd of mi_norm_rows on
    it, bit for bit, and leaves its hand-off words empty (two launches in a row, the second
    with fewer rows)."""
    mo = Moe(7, E=E, hidden=hidden, inter=inter, router_n=E + 16)
    print(f"down_norm E={E} hidden={hidden} inter={inter} M={M}", flush=True)
    rng = np.random.default_rng(70 + M)
    handoff = empty((M, hidden // 2), np.uint32)
    mi.call("mi_gemv_handoff_init", ptr(handoff), M * hidden // 2, stream())
    w = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    dw = dev(w)
    for rows in (M, max(1, M - 1)):
        lg = rng.standard_normal((rows, mo.router_n)).astype(np.float32)
        x = O.f32_to_f16_bits(rng.standard_normal((rows, hidden)).astype(np.float32))
        resid = O.f32_to_f16_bits(rng.standard_normal((rows, hidden)).astype(np.float32))
        dl, dx = dev(lg), dev(x)
        route = empty((rows, ROUTE_WORDS), np.uint32)
        h = empty((rows, mo.top_k + 1, inter), np.uint16)
        mi.call("mi_moe_route", ptr(dl), ptr(route), rows, E, mo.top_k, mo.router_n, stream())
        mi.call("mi_moe_gate_up", ptr(route), ptr(dx), ptr(mo.d_gu), ptr(h), rows, E, mo.top_k, hidden, inter,
                stream())
        r1, r2 = dev(resid), dev(resid)
        x1, x2 = empty((rows, hidden), np.uint16), empty((rows, hidden), np.uint16)
        s1, s2 = empty((rows,), np.float32), empty((rows,), np.float32)
        status = dev(np.zeros(1, np.uint32))
        mi.call("mi_moe_down", ptr(route), ptr(h), ptr(mo.d_dn), ptr(r1), rows, E, mo.top_k, hidden, inter, stream())
        mi.call("mi_norm_rows", ptr(r1), ptr(dw), ptr(x1), ptr(s1), rows, hidden, np.float32(1e-6), stream())
        mi.call("mi_moe_down_norm", ptr(route), ptr(h), ptr(mo.d_dn), ptr(r2), rows, E, mo.top_k, hidden, inter,
                ptr(dw), ptr(x2), ptr(s2), np.float32(1e-6), ptr(handoff), ptr(status), 0, 0, stream())
        sync()
        assert host(status, np.uint32)[0] == 0
        assert np.all(host(handoff, np.uint32) == 0xFFFFFFFF), "hand-off words not left empty"
        assert np.array_equal(host(r1, np.uint16), host(r2, np.uint16))
        assert np.array_equal(host(x1, np.uint16), host(x2, np.uint16))
        assert np.array_equal(host(s1, np.uint32), host(s2, np.uint32))
    # the timeout path, forced from the host: the down work-groups publish nothing and the
    # norm's waits give up after 64 polls; every kernel ends, the status word says so, and the
    # hand-off words are left empty for the next launch
    status = dev(np.zeros(1, np.uint32))
    mi.call("mi_moe_down_norm", ptr(route), ptr(h), ptr(mo.d_dn), ptr(dev(resid)), rows, E, mo.top_k, hidden,
            inter, ptr(dw), ptr(x2), ptr(s2), np.float32(1e-6), ptr(handoff), ptr(status), 64, 1, stream())
    sync()
    assert host(status, np.uint32)[0] == 0xDEAD0003
    assert np.all(host(handoff, np.uint32) == 0xFFFFFFFF)


def test_malformed_route_row_reads_the_shared_block():
    mo = Moe(2, E=16, hidden=512, inter=128, router_n=32)
    M = 1
    x = O.f32_to_f16_bits(np.random.default_rng(0).standard_normal((M, mo.hidden)).astype(np.float32))
    bad = np.zeros((M, ROUTE_WORDS), np.uint32)
    bad[0, :8] = 0xFFFFFFF0  # ids far past the weights
    bad[0, 8:16] = np.float32(0.125).view(np.uint32)
    bad[0, 16] = np.float32(0.5).view(np.uint32)
    dr, dx = dev(bad), dev(x)
    h = empty((M, mo.top_k + 1, mo.inter), np.uint16)
    mi.call("mi_moe_gate_up", ptr(dr), ptr(dx), ptr(mo.d_gu), ptr(h), M, mo.E, mo.top_k, mo.hidden, mo.inter,
            stream())
    sync()
    hh = host(h, np.uint16)
    # every slot computed the shared expert's block
    for slot in range(mo.top_k):
        assert np.array_equal(hh[0, slot], hh[0, mo.top_k])


@pytest.mark.parametrize("T,bad", [(1, False), (37, True), (300, False)])
def test_moe_prefill_matches_decode_kernels(T, bad):
    """mi_moe_prefill (the chunk's expert FFN grouped by expert on the MFMA tile) against the
    oracle of the prefill block (orc_moe_prefill, pf_moe_ref.h's values) at rel 2e-3, and
    against the decode kernels (mi_moe_gate_up + mi_moe_down) on the same route rows within 2 %
    of the largest output (the prefill rounds each dequantised weight to fp16, the decode
    kernels multiply exact integers and scale per group). The router GEMV and the route over all T rows
    in one launch are bitwise the 16-row launches. bad: some route ids outside [0, E), which
    both paths send to the shared expert."""
    mo = Moe(11)
    E, K, H, I = mo.E, mo.top_k, mo.hidden, mo.inter
    rng = np.random.default_rng(T)
    x = O.f32_to_f16_bits(rng.standard_normal((T, H)).astype(np.float32))
    dx = dev(x)
    logits = empty((T, mo.router_n), np.float32)
    route = empty((T, ROUTE_WORDS), np.uint32)
    print(f"moe_prefill T={T}", flush=True)
    mi.call("mi_gemv_f16w", ptr(mo.d_router), ptr(dx), ptr(logits), T, H, mo.router_n, 16, stream())
    mi.call("mi_moe_route", ptr(logits), ptr(route), T, E, K, mo.router_n, stream())
    sync()
    lg_all, rt_all = host(logits, np.float32).reshape(T, -1), host(route, np.uint32).reshape(T, -1)
    for r0 in range(0, T, 16):
        m = min(16, T - r0)
        ls, rs = empty((m, mo.router_n), np.float32), empty((m, ROUTE_WORDS), np.uint32)
        xs = dev(x[r0:r0 + m])
        mi.call("mi_gemv_f16w", ptr(mo.d_router), ptr(xs), ptr(ls), m, H, mo.router_n, 16, stream())
        mi.call("mi_moe_route", ptr(ls), ptr(rs), m, E, K, mo.router_n, stream())
        sync()
        assert np.array_equal(host(ls, np.float32).reshape(m, -1), lg_all[r0:r0 + m])
        assert np.array_equal(host(rs, np.uint32).reshape(m, -1), rt_all[r0:r0 + m])
    if bad:
        rt_all[::5, 2] = E + 5
        rt_all[3, 0] = 0xFFFFFFFF
    droute = dev(np.ascontiguousarray(rt_all))
    # the decode kernels, 16 rows at a time
    want = np.zeros((T, H), np.uint16)
    for r0 in range(0, T, 16):
        m = min(16, T - r0)
        h = empty((m, K + 1, I), np.uint16)
        res = dev(np.zeros((m, H), np.uint16))
        rs = dev(np.ascontiguousarray(rt_all[r0:r0 + m]))
        xs = dev(x[r0:r0 + m])
        mi.call("mi_moe_gate_up", ptr(rs), ptr(xs), ptr(mo.d_gu), ptr(h), m, E, K, H, I, stream())
        mi.call("mi_moe_down", ptr(rs), ptr(h), ptr(mo.d_dn), ptr(res), m, E, K, H, I, stream())
        sync()
        want[r0:r0 + m] = host(res, np.uint16).reshape(m, H)
    # the grouped path
    P = T * (K + 1)
    lst, tiles, tiles_n = empty(P, np.uint32), empty(((P + 63) // 64 + E + 1) * 4, np.uint32), empty(1, np.uint32)
    hh, dd = empty((P, I), np.uint16), empty((P, H), np.uint16)
    resid = dev(np.zeros((T, H), np.uint16))
    mi.call("mi_moe_prefill", ptr(droute), ptr(dx), ptr(mo.d_gu), ptr(mo.d_dn), ptr(resid), T, E, K, H, I, ptr(lst),
            ptr(tiles), ptr(tiles_n), ptr(hh), ptr(dd), stream())
    sync()
    got = O.f16_bits_to_f32(host(resid, np.uint16).reshape(T, H)).astype(np.float64)
    ref = O.f16_bits_to_f32(want).astype(np.float64)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - ref)) <= 0.02 * np.max(np.abs(ref)), np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    # the oracle of the prefill block (tests/kernels/pf_moe_ref.h's values, pinned bit for bit to
    # the reference's twin): rel 2e-3 on every row whose ids are all valid (the reference clamps
    # a bad id to the last expert where this build reads the shared expert)
    orc = np.zeros((T, H), np.uint16)
    O.lib().orc_moe_prefill(O.ORC_F16, E, K, H, I, O._p(np.ascontiguousarray(rt_all)), O._p(x), O._p(mo.gu),
                            O._p(mo.dn), O._p(orc), T)
    ok = np.all(rt_all[:, :K] < E, axis=1)
    w = O.f16_bits_to_f32(orc).astype(np.float64)[ok]
    g = got[ok]
    assert np.all(np.abs(g - w) <= 2e-3 * np.abs(w) + 2e-3 * np.abs(w).max()), np.abs(g - w).max() / np.abs(w).max()
    # every pair listed once, grouped by expert in ascending (token, slot) order: the stable sort
    # of the pairs by expert (a bad id reads the shared expert E)
    n_tiles = int(host(tiles_n, np.uint32)[0])
    ids = rt_all[:, :K].astype(np.int64)
    ex = np.concatenate([np.where(ids < E, ids, E), np.full((T, 1), E)], axis=1).ravel()
    assert np.array_equal(host(lst, np.uint32), np.argsort(ex, kind="stable").astype(np.uint32))
    assert 1 <= n_tiles <= (P + 63) // 64 + E + 1


def test_moe_prefill_refuses_bad_shapes():
    with pytest.raises(mi.MiError):
        mi.call("mi_moe_prefill", 16, 16, 16, 16, 16, 2049, 256, 8, 2048, 512, 16, 16, 16, 16, 16, None)
    with pytest.raises(mi.MiError):
        mi.call("mi_moe_prefill", 16, 16, 16, 16, 16, 4, 100, 8, 2048, 512, 16, 16, 16, 16, 16, None)

