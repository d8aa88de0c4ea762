"""Pins the oracle's whole dense decode step (orc_dense_step: the layer walk of
src/runtime/capture.cc:997, 1247-1263, 1370-1423, 1461-1480) against an independent fp64
forward of the same model written here from the model's definition: RMSNorm, q/k-norm,
half-split RoPE, GQA softmax attention over positions 0..pos, interleave16 SwiGLU
(src/common/repack.h:64-73), two residual adds per layer, final norm, int4 lm_head.

The per-kernel pieces are pinned bit-exactly elsewhere; this test catches wiring mistakes
that those cannot see (a transposed operand, a wrong residual, a mis-indexed KV row or head
group). Bar: fp16 activations round at every kernel boundary, so the oracle's logits sit
within 5e-3 of the largest fp64 logit (measured: 1e-3) and correlate > 0.9999; the argmax agrees unless the
fp64 top two are closer than that."""
import ctypes as C

import numpy as np
import pytest

import oracle as O

F16 = O.ORC_F16


def f16(a):
    return O.f32_to_f16_bits(np.asarray(a, np.float32))


class TinyModel:
    def __init__(self, seed, layers=2, H=256, QH=4, KVH=2, HD=64, rot=64, I=256, V=512, L=64,
                 qk_norm=True, theta=1e4, act=F16):
        rng = np.random.default_rng(seed)
        self.act = act
        a16 = f16 if act == F16 else (lambda v: O.f32_to_bf16_bits(np.asarray(v, np.float32)))
        self.d = dict(layers=layers, H=H, QH=QH, KVH=KVH, HD=HD, rot=rot, I=I, V=V, L=L, qk_norm=qk_norm)
        self.keep = []
        self.lin = []
        dims = [(H, (QH + 2 * KVH) * HD), (QH * HD, H), (H, 2 * I), (I, H)]
        S = [2, 2, 2, 2]
        layers_c = (O.Layer * layers)()
        self.w = []
        for li in range(layers):
            ws = {}
            lins = []
            for (K, N), s in zip(dims, S):
                q = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
                sc = f16(rng.uniform(0.004, 0.03, (K // 64, N)))
                self.keep += [q, sc]
                lins.append(O.Linear(q.ctypes.data, sc.ctypes.data, K, N, s))
                ws[len(ws)] = O.int4_dequant(q, sc, K, N).astype(np.float64)
            Ly = layers_c[li]
            Ly.qkv, Ly.o, Ly.gate_up, Ly.down = lins
            norms = {}
            for name, n in (("in_norm", H), ("post_norm", H), ("q_norm", HD), ("k_norm", HD)):
                a = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
                self.keep.append(a)
                norms[name] = a
                if name in ("q_norm", "k_norm") and not qk_norm:
                    continue
                setattr(Ly, name, a.ctypes.data)
            ws["norms"] = norms
            self.w.append(ws)
        self.embed = a16(rng.standard_normal((V, H)))
        self.fnorm = (1.0 + 0.02 * rng.standard_normal(H)).astype(np.float32)
        lq = rng.integers(0, 2**32, size=(H // 8, V), dtype=np.uint64).astype(np.uint32)
        ls = f16(rng.uniform(0.004, 0.03, (H // 64, V)))
        self.lm = O.int4_dequant(lq, ls, H, V).astype(np.float64)
        self.rope = O.rope_table(theta, rot, L)
        self.keep += [self.embed, self.fnorm, lq, ls, self.rope, layers_c]
        sh = O.attn_shape(QH, KVH, HD, rot_dim=rot)
        self.m = O.DenseModel(layers, H, I, V, V, L, sh, 1e-6, C.cast(layers_c, C.c_void_p),
                              self.embed.ctypes.data, self.fnorm.ctypes.data,
                              O.Linear(lq.ctypes.data, ls.ctypes.data, H, V, 2), self.rope.ctypes.data, 4,
                              H // 64)
        self.kv_k = a16(rng.standard_normal((layers, KVH, L, HD)))
        self.kv_v = a16(rng.standard_normal((layers, KVH, L, HD)))

    def oracle_step(self, tok, pos):
        kk, vv = self.kv_k.copy(), self.kv_v.copy()
        logits = np.zeros(self.d["V"], np.float32)
        am = O.lib().orc_dense_step(self.act, C.byref(self.m), tok, pos, O._p(kk), O._p(vv), O._p(logits),
                                    self.d["layers"])
        return int(am), logits, kk, vv

    def fp64_step(self, tok, pos, mistake=None, cache=None):
        """cache: the fp64 K and V rows to attend over (default: the model's fp16 cache)"""
        d = self.d
        H, QH, KVH, HD, rot, I = d["H"], d["QH"], d["KVH"], d["HD"], d["rot"], d["I"]
        eps = 1e-6

        def rms(v, w):
            return v / np.sqrt(np.mean(v * v) + eps) * w

        half = rot // 2
        cos = self.rope[pos, 0].astype(np.float64)
        sin = self.rope[pos, 1].astype(np.float64)

        def rope(v):
            out = v.copy()
            a, b = v[:half], v[half:rot]
            out[:half] = a * cos - b * sin if mistake != "rope_sign" else a * cos + b * sin
            out[half:rot] = b * cos + a * sin
            return out

        resid = O.widen(self.act, self.embed[tok]).astype(np.float64)
        if cache is None:
            kc = O.widen(self.act, self.kv_k).astype(np.float64)
            vc = O.widen(self.act, self.kv_v).astype(np.float64)
        else:
            kc, vc = cache[0].copy(), cache[1].copy()
        G = QH // KVH
        for li, ws in enumerate(self.w):
            nm = ws["norms"]
            x = rms(resid, nm["in_norm"])
            qkv = x @ ws[0]
            q = qkv[:QH * HD].reshape(QH, HD)
            k = qkv[QH * HD:(QH + KVH) * HD].reshape(KVH, HD)
            v = qkv[(QH + KVH) * HD:].reshape(KVH, HD)
            if d["qk_norm"]:
                q = np.stack([rms(h, nm["q_norm"]) for h in q])
                k = np.stack([rms(h, nm["k_norm"]) for h in k])
            q = np.stack([rope(h) for h in q])
            k = np.stack([rope(h) for h in k])
            kc[li, :, pos] = k
            vc[li, :, pos] = v
            att = np.empty((QH, HD))
            for h in range(QH):
                kvh = h // G if mistake != "gqa_map" else h % KVH
                sc = kc[li, kvh, :pos + 1] @ q[h] / np.sqrt(HD)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ vc[li, kvh, :pos + 1]
            resid = resid + att.reshape(-1) @ ws[1] if mistake != "no_attn_resid" else att.reshape(-1) @ ws[1]
            x = rms(resid, nm["post_norm"])
            gu = x @ ws[2]
            j = np.arange(I)
            g = gu[(j // 16) * 32 + j % 16]
            u = gu[(j // 16) * 32 + j % 16 + 16]
            if mistake == "gate_up_swap":
                g, u = u, g
            h_ = g / (1.0 + np.exp(-g)) * u
            resid = resid + h_ @ ws[3]
        x = rms(resid, self.fnorm)
        return x @ self.lm, kc, vc


@pytest.mark.parametrize("seed,pos,qk_norm,act", [(1, 0, True, F16), (2, 37, True, F16), (3, 63, False, F16),
                                                  (4, 21, True, O.ORC_BF16), (5, 63, False, O.ORC_BF16)])
def test_dense_step_vs_independent_fp64_forward(seed, pos, qk_norm, act):
    """act: the reference's own bf16 activations too (rne_bf16 at every rounding point, bf16
    embeddings and cache); bf16 keeps 3 bits fewer than f16, so its bars are 8x wider (measured
    errors: f16 ~1e-3, bf16 ~6e-3 of the largest logit)."""
    m = TinyModel(seed, qk_norm=qk_norm, act=act)
    wide = 8.0 if act == O.ORC_BF16 else 1.0
    tok = (seed * 97) % m.d["V"]
    am, got, kk, vv = m.oracle_step(tok, pos)
    want, kc, vc = m.fp64_step(tok, pos)
    scale = np.abs(want).max()
    err = np.abs(got.astype(np.float64) - want)
    print(f"act {act}: max err {err.max() / scale:.2e} of the largest logit")
    assert err.max() <= 5e-3 * wide * scale, (err.max(), scale)
    assert np.corrcoef(got, want)[0, 1] > 1 - 1e-4 * wide
    top = np.sort(want)[::-1]
    assert am == int(np.argmax(want)) or top[0] - want[am] <= 1e-2 * wide * scale
    # the step wrote this position's K and V rows (fp16 of the fp64 values, to the same bar),
    # and nothing else
    for li in range(m.d["layers"]):
        gk = O.widen(act, kk[li, :, pos]).astype(np.float64)
        assert np.abs(gk - kc[li, :, pos]).max() <= 2e-2 * wide * np.abs(kc[li, :, pos]).max()
        gv = O.widen(act, vv[li, :, pos]).astype(np.float64)
        assert np.abs(gv - vc[li, :, pos]).max() <= 2e-2 * wide * np.abs(vc[li, :, pos]).max()
    mask = np.ones(m.d["L"], bool)
    mask[pos] = False
    assert np.array_equal(kk[:, :, mask], m.kv_k[:, :, mask])
    assert np.array_equal(vv[:, :, mask], m.kv_v[:, :, mask])


@pytest.mark.parametrize("act", [F16, O.ORC_BF16])
@pytest.mark.parametrize("mistake", ["rope_sign", "gqa_map", "gate_up_swap", "no_attn_resid"])
def test_bar_rejects_plausible_wiring_mistakes(mistake, act):
    """The comparison is not vacuous: the same fp64 forward with one plausible mistake
    (RoPE sign, GQA head mapping, gate/up swapped, a dropped residual) misses the bar (the bf16
    walk's 8x wider one too)."""
    m = TinyModel(2, act=act)
    wide = 8.0 if act == O.ORC_BF16 else 1.0
    _, got, _, _ = m.oracle_step(194, 37)
    want = m.fp64_step(194, 37, mistake=mistake)[0]
    assert np.abs(got - want).max() > 5e-3 * wide * np.abs(want).max()


def prefill_fp64(m, ids, pos, mistake=None):
    """T consecutive fp64 steps (each attending to the fp64 K/V rows of the previous ones)"""
    cache = (O.f16_bits_to_f32(m.kv_k).astype(np.float64), O.f16_bits_to_f32(m.kv_v).astype(np.float64))
    for t, tok in enumerate(ids):
        lg, kc, vc = m.fp64_step(int(tok), pos + t, mistake=mistake, cache=cache)
        cache = (kc, vc)
    return lg, cache[0], cache[1]


def oracle_prefill(m, ids, pos):
    kk, vv = m.kv_k.copy(), m.kv_v.copy()
    logits = np.zeros(m.d["V"], np.float32)
    ids = np.ascontiguousarray(ids, np.uint32)
    am = O.lib().orc_prefill_chunk(F16, C.byref(m.m), O._p(ids), len(ids), pos, O._p(kk), O._p(vv), O._p(logits))
    return int(am), logits, kk, vv


@pytest.mark.parametrize("seed,T,pos,qk_norm", [(4, 12, 0, True), (5, 23, 30, True), (6, 9, 50, False)])
def test_prefill_chunk_vs_independent_fp64_forward(seed, T, pos, qk_norm):
    """orc_prefill_chunk (the prefill walk with its own roundings: weights rounded once, fp32
    sums, fp64 attention rounded once) against T consecutive fp64 steps of the same model: the
    last row's logits and every K/V row the chunk writes, at the step's bar, and nothing else
    of the cache touched."""
    m = TinyModel(seed, qk_norm=qk_norm)
    ids = np.random.default_rng(seed).integers(0, m.d["V"], T)
    am, got, kk, vv = oracle_prefill(m, ids, pos)
    want, kc, vc = prefill_fp64(m, ids, pos)
    scale = np.abs(want).max()
    err = np.abs(got.astype(np.float64) - want)
    assert err.max() <= 5e-3 * scale, (err.max(), scale)
    assert np.corrcoef(got, want)[0, 1] > 0.9999
    top = np.sort(want)[::-1]
    assert am == int(np.argmax(want)) or top[0] - want[am] <= 1e-2 * scale
    rows = slice(pos, pos + T)
    for li in range(m.d["layers"]):
        gk = O.f16_bits_to_f32(kk[li, :, rows]).astype(np.float64)
        assert np.abs(gk - kc[li, :, rows]).max() <= 2e-2 * np.abs(kc[li, :, rows]).max()
        gv = O.f16_bits_to_f32(vv[li, :, rows]).astype(np.float64)
        assert np.abs(gv - vc[li, :, rows]).max() <= 2e-2 * np.abs(vc[li, :, rows]).max()
    mask = np.ones(m.d["L"], bool)
    mask[rows] = False
    assert np.array_equal(kk[:, :, mask], m.kv_k[:, :, mask])
    assert np.array_equal(vv[:, :, mask], m.kv_v[:, :, mask])


@pytest.mark.parametrize("mistake", ["rope_sign", "gqa_map", "gate_up_swap", "no_attn_resid"])
def test_prefill_bar_rejects_plausible_wiring_mistakes(mistake):
    m = TinyModel(5)
    ids = np.random.default_rng(5).integers(0, m.d["V"], 10)
    _, got, _, _ = oracle_prefill(m, ids, 20)
    want = prefill_fp64(m, ids, 20, mistake=mistake)[0]
    assert np.abs(got - want).max() > 5e-3 * np.abs(want).max()


def test_prefill_chunk_refuses_what_it_does_not_model():
    m = TinyModel(4)
    logits = np.zeros(m.d["V"], np.float32)
    ids = np.zeros(4, np.uint32)
    kk, vv = m.kv_k.copy(), m.kv_v.copy()
    # past the cache
    assert O.lib().orc_prefill_chunk(F16, C.byref(m.m), O._p(ids), 4, m.d["L"] - 2, O._p(kk), O._p(vv),
                                     O._p(logits)) == 0xFFFFFFFF


def layout1_dequant(blocks, K, N):
    """fp64 [K][N] of one int4 g64 layout-1 block, from the format's definition: tile
    (n/16, k/64) of 136 words; word (k%64)/8 * 16 + n%16 holds k's nibble k%8 (low first);
    the 16 fp16 scales follow the 128 nibble words."""
    G, NT = K // 64, N // 16
    t = blocks[:NT * G * 136].reshape(NT, G, 136)
    nib = (t[:, :, :128].reshape(NT, G, 8, 16)[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    # nib [nt][g][j][n16][i] -> k = g*64 + j*8 + i, n = nt*16 + n16
    q = nib.astype(np.float64) - 8.0
    sc = O.f16_bits_to_f32(t[:, :, 128:].copy().view(np.uint16).reshape(NT, G, 16)).astype(np.float64)
    w = q * sc[:, :, None, :, None]
    return w.transpose(1, 2, 4, 0, 3).reshape(K, N)


class TinyMoe(TinyModel):
    """TinyModel whose MLPs are the MoE block: E routed experts, top_k + a shared one."""

    def __init__(self, seed, E=16, top_k=4, moe_inter=128, H=512, **kw):
        super().__init__(seed, H=H, I=256, **kw)
        rng = np.random.default_rng(seed + 1000)
        self.E, self.top_k, self.mi_ = E, top_k, moe_inter
        self.router_n = (E + 1 + 15) // 16 * 16
        layers_c = C.cast(self.m.layer, C.POINTER(O.Layer))
        gub = (2 * moe_inter // 16) * (H // 64) * 136
        dnb = (H // 16) * (moe_inter // 64) * 136
        for li in range(self.d["layers"]):
            rw = np.zeros((self.router_n, H), np.float32)
            rw[:E + 1] = 0.05 * rng.standard_normal((E + 1, H))
            rw16 = f16(rw)
            rt = np.empty(self.router_n * H, np.uint16)
            O.lib().orc_f16w_tile(O._p(rw16), H, self.router_n, O._p(rt))

            def blocks(n_blocks, K, N):
                tiles = n_blocks * (N // 16) * (K // 64)
                b = rng.integers(0, 2**32, size=(tiles, 136), dtype=np.uint64).astype(np.uint32)
                b[:, 128:] = f16(rng.uniform(0.004, 0.03, (tiles, 16))).view(np.uint32).reshape(tiles, 8)
                return b.reshape(-1)
            gu, dn = blocks(E + 1, H, 2 * moe_inter), blocks(E + 1, moe_inter, H)
            self.keep += [rt, gu, dn]
            L = layers_c[li]
            L.router, L.moe_gu, L.moe_dn = rt.ctypes.data, gu.ctypes.data, dn.ctypes.data
            self.w[li]["router"] = O.f16_bits_to_f32(rw16).astype(np.float64)
            self.w[li]["gu"] = [layout1_dequant(gu[e * gub:(e + 1) * gub], H, 2 * moe_inter) for e in range(E + 1)]
            self.w[li]["dn"] = [layout1_dequant(dn[e * dnb:(e + 1) * dnb], moe_inter, H) for e in range(E + 1)]
        self.m.experts, self.m.top_k, self.m.moe_inter = E, top_k, moe_inter
        self.m.router_n, self.m.router_ksplit = self.router_n, 16
        self.ids = []

    def mlp(self, ws, x, mistake=None):
        E, k = self.E, self.top_k
        lg = ws["router"] @ x
        p = np.exp(lg[:E] - lg[:E].max())
        p /= p.sum()
        ids = sorted(range(E), key=lambda e: (-p[e], e))[:k]
        self.ids.append(ids)
        w = p[ids] / p[ids].sum()
        j = np.arange(self.mi_)

        def expert(e):
            gu = x @ ws["gu"][e]
            g, u = gu[(j // 16) * 32 + j % 16], gu[(j // 16) * 32 + j % 16 + 16]
            if mistake == "moe_gate_up_swap":
                g, u = u, g
            return (g / (1.0 + np.exp(-g)) * u) @ ws["dn"][e]
        out = sum(wk * expert(e) for wk, e in zip(w, ids))
        sg = 1.0 / (1.0 + np.exp(-lg[E]))
        return out + (sg if mistake != "moe_no_shared" else 0.0) * expert(E)


def _fp64_moe_step(m, tok, pos, mistake=None):
    """TinyModel.fp64_step with each layer's MLP replaced by TinyMoe.mlp."""
    orig = m.w
    d = m.d
    H, QH, KVH, HD = d["H"], d["QH"], d["KVH"], d["HD"]
    eps = 1e-6

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v) + eps) * w
    half = d["rot"] // 2
    cos, sin = m.rope[pos, 0].astype(np.float64), m.rope[pos, 1].astype(np.float64)

    def rope(v):
        out = v.copy()
        a, b = v[:half], v[half:d["rot"]]
        out[:half] = a * cos - b * sin
        out[half:d["rot"]] = b * cos + a * sin
        return out
    resid = O.f16_bits_to_f32(m.embed[tok]).astype(np.float64)
    kc = O.f16_bits_to_f32(m.kv_k).astype(np.float64)
    vc = O.f16_bits_to_f32(m.kv_v).astype(np.float64)
    G = QH // KVH
    for li, ws in enumerate(orig):
        nm = ws["norms"]
        x = rms(resid, nm["in_norm"])
        qkv = x @ ws[0]
        q = qkv[:QH * HD].reshape(QH, HD)
        k = qkv[QH * HD:(QH + KVH) * HD].reshape(KVH, HD)
        v = qkv[(QH + KVH) * HD:].reshape(KVH, HD)
        q = np.stack([rope(rms(h, nm["q_norm"])) for h in q])
        k = np.stack([rope(rms(h, nm["k_norm"])) for h in k])
        kc[li, :, pos], vc[li, :, pos] = k, v
        att = np.empty((QH, HD))
        for h in range(QH):
            sc = kc[li, h // G, :pos + 1] @ q[h] / np.sqrt(HD)
            p = np.exp(sc - sc.max())
            att[h] = (p / p.sum()) @ vc[li, h // G, :pos + 1]
        resid = resid + att.reshape(-1) @ ws[1]
        resid = resid + m.mlp(ws, rms(resid, nm["post_norm"]), mistake)
    return rms(resid, m.fnorm) @ m.lm


@pytest.mark.parametrize("seed,pos", [(7, 0), (8, 33)])
def test_moe_step_vs_independent_fp64_forward(seed, pos):
    m = TinyMoe(seed)
    tok = seed * 13
    am, got, _, _ = m.oracle_step(tok, pos)
    want = _fp64_moe_step(m, tok, pos)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 5e-3 * scale, np.abs(got - want).max() / scale
    assert np.corrcoef(got, want)[0, 1] > 0.9999


@pytest.mark.parametrize("mistake", ["moe_gate_up_swap", "moe_no_shared"])
def test_moe_bar_rejects_plausible_mistakes(mistake):
    m = TinyMoe(7)
    _, got, _, _ = m.oracle_step(91, 33)
    want = _fp64_moe_step(m, 91, 33, mistake)
    assert np.abs(got - want).max() > 5e-3 * np.abs(want).max()


SIGN_WORDS = [0xA197D809, 0xA6850592, 0xB205A73E, 0x20AFA769, 0x45C2CF64, 0xBEAEAACB, 0x75F39ADD, 0x2385A70C]


def unrotate64(y):
    """R^T in fp64 along the last axis (R = H_256 diag(s) / 16, src/common/kv8.h:1-26)."""
    from scipy.linalg import hadamard
    s = np.array([-1.0 if (SIGN_WORDS[j >> 5] >> (j & 31)) & 1 else 1.0 for j in range(256)])
    return (y * s) @ hadamard(256).astype(np.float64) / 16.0


class TinyKv8(TinyModel):
    """TinyModel with head_dim 256 and the int8 rotated KV cache: rows [0, L) hold the
    writer's encoding of N(0, 1) fp16 rows."""

    def __init__(self, seed, **kw):
        super().__init__(seed, H=256, QH=4, KVH=2, HD=256, rot=64, **kw)
        rng = np.random.default_rng(seed + 77)
        d = self.d
        shape = (d["layers"], d["KVH"], d["L"])
        self.k8 = np.zeros(shape + (256,), np.int8)
        self.v8 = np.zeros_like(self.k8)
        self.ks = np.zeros(shape, np.uint16)
        self.vs = np.zeros_like(self.ks)
        for idx in np.ndindex(*shape):
            for c8, cs in ((self.k8, self.ks), (self.v8, self.vs)):
                x = np.ascontiguousarray(O.f16_bits_to_f32(f16(rng.standard_normal(256))))
                cs[idx] = O.lib().orc_kv8_encode256(O._p(x), O._p(c8[idx]))

    def oracle_step_kv8(self, tok, pos):
        k8, v8, ks, vs = self.k8.copy(), self.v8.copy(), self.ks.copy(), self.vs.copy()
        logits = np.zeros(self.d["V"], np.float32)
        am = O.lib().orc_dense_step_kv8(F16, C.byref(self.m), tok, pos, O._p(k8), O._p(v8), O._p(ks), O._p(vs),
                                        O._p(logits), self.d["layers"])
        return int(am), logits, (k8, v8, ks, vs)

    def dequant(self, c8, cs):
        return c8.astype(np.float64) * O.f16_bits_to_f32(cs).astype(np.float64)[..., None]

    def fp64_step_kv8(self, tok, pos, mistake=None):
        """The fp64 forward over the cache in the model's own basis: a cached row's value
        is the un-rotation of its dequantised int8 row (q.k and sum p v are invariant under
        the orthogonal R); the current position's K and V are the exact fp64 values."""
        kd, vd = self.dequant(self.k8, self.ks), self.dequant(self.v8, self.vs)
        if mistake != "kv8_rotated_basis":
            kd, vd = unrotate64(kd), unrotate64(vd)
        return self.fp64_step(tok, pos, cache=(kd, vd))


@pytest.mark.parametrize("seed,pos", [(4, 0), (5, 41)])
def test_kv8_step_vs_independent_fp64_forward(seed, pos):
    """orc_dense_step_kv8 (attn_prep_kv8 + the int8 reader + the rotated reduce in the layer
    walk) against the fp64 forward in the un-rotated basis; the written rows decode, after
    un-rotation, to the step's K and V within the int8 quantiser's bound."""
    m = TinyKv8(seed)
    tok = seed * 31
    am, got, (k8, v8, ks, vs) = m.oracle_step_kv8(tok, pos)
    want, kc, vc = m.fp64_step_kv8(tok, pos)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 5e-3 * scale, np.abs(got - want).max() / scale
    assert np.corrcoef(got, want)[0, 1] > 0.9999
    for li in range(m.d["layers"]):
        for c8, cs, ref in ((k8, ks, kc), (v8, vs, vc)):
            dec = unrotate64(m.dequant(c8[li, :, pos], cs[li, :, pos]))
            step = O.f16_bits_to_f32(cs[li, :, pos])  # the rows' scales
            # per element in the rotated basis |err| <= scale / 2 (+ the 16-bit rounding of
            # the row); R is orthogonal, so the row's 2-norm error is at most 16 * scale / 2
            err = np.linalg.norm(dec - ref[li, :, pos], axis=-1)
            bound = 16 * step.astype(np.float64) / 2 + 2e-3 * np.linalg.norm(ref[li, :, pos], axis=-1)
            assert np.all(err <= bound), (err, bound)
    mask = np.ones(m.d["L"], bool)
    mask[pos] = False
    assert np.array_equal(k8[:, :, mask], m.k8[:, :, mask]) and np.array_equal(vs[:, :, mask], m.vs[:, :, mask])


def test_kv8_bar_rejects_a_missing_unrotation():
    m = TinyKv8(5)
    _, got, _ = m.oracle_step_kv8(155, 41)
    want = m.fp64_step_kv8(155, 41, mistake="kv8_rotated_basis")[0]
    assert np.abs(got - want).max() > 5e-3 * np.abs(want).max()


class TinyMtp(TinyModel):
    """TinyModel plus an MTP head (capture.cc:1772-1939): fc [2H] -> H, one dense decoder
    layer with its own one-layer KV cache, the embedding / hidden / final norms; the head
    shares the model's embedding and lm_head."""

    def __init__(self, seed, w16=False, **kw):
        super().__init__(seed, **kw)
        d = self.d
        H, QH, KVH, HD, I, L = d["H"], d["QH"], d["KVH"], d["HD"], d["I"], d["L"]
        rng = np.random.default_rng(seed + 500)
        w16s = []  # w16: the linears' f16 [N][K] matrices in orc_f16w_tile's layout

        def lin(K, N, S=2):
            if w16:
                w = f16(rng.standard_normal((N, K)) * 0.06)
                t = np.zeros_like(w)
                O.lib().orc_f16w_tile(O._p(w), K, N, O._p(t))
                self.keep.append(t)
                w16s.append(t.ctypes.data)
                return O.Linear(None, None, 0, 0, 0), O.f16_bits_to_f32(w).astype(np.float64).T
            q = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
            sc = f16(rng.uniform(0.004, 0.03, (K // 64, N)))
            self.keep += [q, sc]
            return O.Linear(q.ctypes.data, sc.ctypes.data, K, N, S), O.int4_dequant(q, sc, K, N).astype(np.float64)

        def gamma(n):
            a = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
            self.keep.append(a)
            return a

        self.hw = {}
        fc, self.hw["fc"] = lin(2 * H, H)
        Ly = O.Layer()
        lins = []
        for i, (K, N) in enumerate([(H, (QH + 2 * KVH) * HD), (QH * HD, H), (H, 2 * I), (I, H)]):
            l, w = lin(K, N)
            lins.append(l)
            self.hw[i] = w
        Ly.qkv, Ly.o, Ly.gate_up, Ly.down = lins
        self.hn = {k: gamma(n) for k, n in (("in_norm", H), ("post_norm", H), ("q_norm", HD), ("k_norm", HD),
                                           ("pre_e", H), ("pre_h", H), ("final", H))}
        Ly.in_norm, Ly.post_norm = self.hn["in_norm"].ctypes.data, self.hn["post_norm"].ctypes.data
        if d["qk_norm"]:
            Ly.q_norm, Ly.k_norm = self.hn["q_norm"].ctypes.data, self.hn["k_norm"].ctypes.data
        self.head = O.MtpHead(fc, Ly, self.hn["pre_e"].ctypes.data, self.hn["pre_h"].ctypes.data,
                              self.hn["final"].ctypes.data, *w16s)
        self.hkv_k = f16(rng.standard_normal((KVH, L, HD)))
        self.hkv_v = f16(rng.standard_normal((KVH, L, HD)))

    def oracle_head(self, tok, h16, p, kk, vv, full=1):
        logits = np.zeros(self.d["V"], np.float32)
        hout = np.zeros(self.d["H"], np.uint16)
        am = O.lib().orc_mtp_head_step(F16, C.byref(self.m), C.byref(self.head), tok, O._p(h16), p, O._p(kk),
                                       O._p(vv), full, O._p(hout), O._p(logits))
        return int(am), logits, hout

    def fp64_head(self, tok, h, p, kc, vc, mistake=None):
        """fp64 forward of the head at position p; h fp64 [H]; kc / vc fp64 [KVH][L][HD]
        (updated at p). Returns (logits, h_out)."""
        d = self.d
        H, QH, KVH, HD, rot, I = d["H"], d["QH"], d["KVH"], d["HD"], d["rot"], d["I"]
        eps = 1e-6

        def rms(v, w):
            return v / np.sqrt(np.mean(v * v) + eps) * w

        half = rot // 2
        rp = p + 1 if mistake == "head_pos" else p
        cos = self.rope[rp, 0].astype(np.float64)
        sin = self.rope[rp, 1].astype(np.float64)

        def rope(v):
            out = v.copy()
            a, b = v[:half], v[half:rot]
            out[:half] = a * cos - b * sin
            out[half:rot] = b * cos + a * sin
            return out

        e = O.f16_bits_to_f32(self.embed[tok]).astype(np.float64)
        halves = [rms(e, self.hn["pre_e"]), rms(h, self.hn["pre_h"])]
        if mistake == "cat_swap":
            halves = halves[::-1]
        resid = np.concatenate(halves) @ self.hw["fc"]
        if mistake == "stale_resid":
            resid = resid + e
        x = rms(resid, self.hn["in_norm"])
        qkv = x @ self.hw[0]
        q = qkv[:QH * HD].reshape(QH, HD)
        k = qkv[QH * HD:(QH + KVH) * HD].reshape(KVH, HD)
        v = qkv[(QH + KVH) * HD:].reshape(KVH, HD)
        if d["qk_norm"]:
            q = np.stack([rms(r, self.hn["q_norm"]) for r in q])
            k = np.stack([rms(r, self.hn["k_norm"]) for r in k])
        q = np.stack([rope(r) for r in q])
        k = np.stack([rope(r) for r in k])
        kc[:, p], vc[:, p] = k, v
        G = QH // KVH
        att = np.empty((QH, HD))
        for hh in range(QH):
            sc = kc[hh // G, :p + 1] @ q[hh] / np.sqrt(HD)
            w = np.exp(sc - sc.max())
            att[hh] = (w / w.sum()) @ vc[hh // G, :p + 1]
        resid = resid + att.reshape(-1) @ self.hw[1]
        x = rms(resid, self.hn["post_norm"])
        gu = x @ self.hw[2]
        j = np.arange(I)
        g, u = gu[(j // 16) * 32 + j % 16], gu[(j // 16) * 32 + j % 16 + 16]
        resid = resid + (g / (1.0 + np.exp(-g)) * u) @ self.hw[3]
        x = rms(resid, self.hn["final"]) if mistake != "no_final_norm" else resid
        return x @ self.lm, x


def _head_case(m, tok, p, seed):
    h = O.f16_bits_to_f32(f16(np.random.default_rng(seed).standard_normal(m.d["H"]))).astype(np.float64)
    return h, f16(h)


@pytest.mark.parametrize("seed,p,qk_norm,w16", [(1, 0, True, False), (2, 29, True, False), (3, 63, False, False),
                                                (4, 0, True, True), (5, 40, True, True), (6, 63, False, True)])
def test_mtp_head_vs_independent_fp64_forward(seed, p, qk_norm, w16):
    """orc_mtp_head_step against an fp64 forward of the head written here: the draft's logits,
    its output hidden and the K/V row it writes at the head position, and two chained drafts
    (the second fed the first's id and output hidden), at the dense step's bar; the fill form
    (full = 0) writes the same K/V row and nothing else. w16: the head's linears as 16-bit
    matrices (the reference's bf16 head, loader.cc:586-597) through orc_gemv_f16w."""
    m = TinyMtp(seed, w16=w16, qk_norm=qk_norm)
    tok = (seed * 131) % m.d["V"]
    h, h16 = _head_case(m, tok, p, seed)
    kk, vv = m.hkv_k.copy(), m.hkv_v.copy()
    kc = O.f16_bits_to_f32(m.hkv_k).astype(np.float64)
    vc = O.f16_bits_to_f32(m.hkv_v).astype(np.float64)
    toks, hs = tok, h16
    for step in range(2 if p + 1 < m.d["L"] else 1):
        am, got, hout = m.oracle_head(toks, hs, p + step, kk, vv)
        want, hwant = m.fp64_head(toks, O.f16_bits_to_f32(hs).astype(np.float64), p + step, kc, vc)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 5e-3 * scale, (step, np.abs(got - want).max(), scale)
        assert np.corrcoef(got, want)[0, 1] > 0.9999
        top = np.sort(want)[::-1]
        assert am == int(np.argmax(want)) or top[0] - want[am] <= 1e-2 * scale
        gh = O.f16_bits_to_f32(hout).astype(np.float64)
        assert np.abs(gh - hwant).max() <= 2e-2 * np.abs(hwant).max()
        for a, b in ((kk, kc), (vv, vc)):
            g = O.f16_bits_to_f32(a[:, p + step]).astype(np.float64)
            assert np.abs(g - b[:, p + step]).max() <= 2e-2 * np.abs(b[:, p + step]).max()
        # the second draft: the id the first drafted and the head's own output hidden
        toks, hs = am, hout
        kc[:, p + step] = O.f16_bits_to_f32(kk[:, p + step])  # the cache as the oracle holds it
        vc[:, p + step] = O.f16_bits_to_f32(vv[:, p + step])
    kf, vf = m.hkv_k.copy(), m.hkv_v.copy()
    assert m.oracle_head(tok, h16, p, kf, vf, full=0)[0] == 0
    assert np.array_equal(kf[:, p], kk[:, p]) and np.array_equal(vf[:, p], vv[:, p])
    mask = np.ones(m.d["L"], bool)
    mask[p] = False
    assert np.array_equal(kf[:, mask], m.hkv_k[:, mask]) and np.array_equal(vf[:, mask], m.hkv_v[:, mask])


@pytest.mark.parametrize("w16", [False, True])
@pytest.mark.parametrize("mistake", ["cat_swap", "stale_resid", "head_pos", "no_final_norm"])
def test_mtp_bar_rejects_plausible_wiring_mistakes(mistake, w16):
    """The head's comparison is not vacuous: the fp64 forward with one plausible mistake (the
    concat halves swapped, the fc output added to a stale residual, the head's RoPE one
    position off, the final norm dropped) misses the bar."""
    m = TinyMtp(2, w16=w16)
    h, h16 = _head_case(m, 77, 29, 2)
    _, got, _ = m.oracle_head(77, h16, 29, m.hkv_k.copy(), m.hkv_v.copy())
    kc = O.f16_bits_to_f32(m.hkv_k).astype(np.float64)
    vc = O.f16_bits_to_f32(m.hkv_v).astype(np.float64)
    want = m.fp64_head(77, h, 29, kc, vc, mistake=mistake)[0]
    assert np.abs(got - want).max() > 5e-3 * np.abs(want).max()
