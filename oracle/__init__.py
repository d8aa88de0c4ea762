"""CPU oracle - TEST INFRASTRUCTURE ONLY.

A ctypes view of ``liboracle.so`` (this repository's C++ restatement of the reference's
scalar host twins, see oracle.h) and, when built, ``_ref/libref.so`` (the reference's own
twins compiled from /root/reference). Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg import this package, and only as the checker: the product
path (the HIP library) never calls it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_BF16, ORC_F16 = 0, 1

_lib = None
_ref = None


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            from . import build_oracle
            build_oracle.build_oracle()
        _lib = C.CDLL(path)
        L = _lib
        u16, u32, f32, i32, sz = C.c_uint16, C.c_uint32, C.c_float, C.c_int, C.c_size_t
        vp = C.c_void_p
        sig = {
            "orc_f32_to_bf16": (u16, [f32]), "orc_bf16_to_f32": (f32, [u16]),
            "orc_f32_to_f16": (u16, [f32]), "orc_f32_to_f16_ftz": (u16, [f32]),
            "orc_f32_to_f16_sat": (u16, [f32]), "orc_f16_to_f32": (f32, [u16]),
            "orc_rne": (u16, [i32, f32]), "orc_widen": (f32, [i32, u16]),
            "orc_int4_dequant": (None, [vp, vp, u32, u32, vp]),
            "orc_repack_layout1": (None, [vp, vp, u32, u32, vp]),
            "orc_interleave16_l0": (None, [vp, vp, vp, vp, u32, u32, vp, vp]),
            "orc_gemv_ref": (None, [u32, vp, vp, u32, u32, vp, u32, vp, vp]),
            "orc_gemv_twin": (None, [u32, vp, vp, u32, u32, vp, u32, u32, vp]),
            "orc_gemv_twin_partials": (None, [u32, vp, vp, u32, u32, vp, u32, u32, vp]),
            "orc_n2_over": (sz, [vp, vp, vp, sz, vp]),
            "orc_res_norm": (None, [i32, vp, vp, vp, vp, u32, u32, u32, f32]),
            "orc_res_fold": (None, [i32, vp, vp, vp, u32, u32, u32, u32]),
            "orc_norm_finish": (None, [i32, vp, vp, vp, vp, u32, u32, u32, f32]),
            "orc_silu_mul": (None, [i32, vp, vp, u32, u32, u32]),
            "orc_rope_table": (None, [C.c_double, u32, u32, vp]),
            "orc_attn_prep": (None, [i32, vp, u32, u32, u32, vp, u32, vp, vp, vp, vp, vp, vp,
                                     vp, sz, sz, vp, u32]),
            "orc_v2_ppw": (u32, [u32, u32]),
            "orc_attn_decode_v2": (None, [i32, vp, u32, u32, u32, u32, vp, u32, vp, vp, vp, vp,
                                          sz, sz, sz, sz, vp, u32, vp]),
            "orc_attn_reduce_v2": (None, [i32, vp, u32, u32, u32, u32, vp, vp, vp]),
            "orc_attend64": (None, [vp, vp, u32, u32, u32, i32, vp, vp, vp, vp, sz, sz, sz, sz,
                                    vp, u32, vp]),
            "orc_kv8_rotate256": (None, [vp, vp]), "orc_kv8_unrotate256": (None, [vp, vp]),
            "orc_kv8_quantise": (u16, [vp, vp, u32]), "orc_kv8_encode256": (u16, [vp, vp]),
            "orc_kv8_dequant": (f32, [C.c_int8, u16]),
            "orc_attn_prep_kv8": (None, [i32, vp, u32, u32, u32, vp, u32, vp, vp, vp, vp, vp, vp,
                                         vp, vp, vp, sz, sz, sz, sz, vp, u32]),
            "orc_attn_reduce_v2_kv8": (None, [i32, vp, u32, u32, u32, u32, vp, vp, vp]),
            "orc_embed_gather": (i32, [vp, u32, vp, u32, u32, vp]),
            "orc_argmax": (u32, [vp, u32, u32]),
            "orc_accept_greedy": (u32, [vp, vp, u32, vp]),
            "orc_moe_route_fn": (None, [i32, vp, u32, u32, vp]),
            "orc_moe_split_dot": (f32, [i32, u32, vp, vp, u32, u32, u32, vp, u32]),
            "orc_moe_silu_up": (u16, [i32, f32, f32]),
            "orc_moe_combine": (u16, [i32, vp, vp, u32, u16]),
            "orc_moe_block": (None, [i32, u32, u32, u32, u32, u32, vp, vp, vp, vp, sz, sz, vp,
                                     vp, sz, sz, u32, u32, vp, vp]),
            "orc_dense_step": (u32, [i32, vp, u32, u32, vp, vp, vp, u32]),
            "orc_dense_step_kv8": (u32, [i32, vp, u32, u32, vp, vp, vp, vp, vp, u32]),
            "orc_prefill_chunk": (u32, [i32, vp, vp, u32, u32, vp, vp, vp]),
            "orc_mtp_head_step": (u32, [i32, vp, vp, u32, vp, u32, vp, vp, i32, vp, vp]),
            "orc_quantise_row_int8": (f32, [vp, u32, vp]),
            "orc_rtn_int4_g64": (None, [vp, u32, u32, vp, vp]),
            "orc_gemv_i8w": (None, [i32, vp, vp, vp, u32, u32, u32, vp]),
            "orc_moe_prefill": (None, [i32, u32, u32, u32, u32, vp, vp, vp, vp, vp, u32]),
            "orc_gemv_f16w": (None, [i32, vp, vp, u32, u32, u32, u32, vp]),
            "orc_f16w_tile": (None, [vp, u32, u32, vp]),
            "orc_threads": (i32, []),
            "orc_set_threads": (None, [i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ref():
    """The reference's own twins (oracle/_ref/libref.so) or None when not built."""
    global _ref
    if _ref is None:
        path = os.path.join(HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        _ref = C.CDLL(path)
        R = _ref
        u16, u32, f32, vp = C.c_uint16, C.c_uint32, C.c_float, C.c_void_p
        sig = {
            "ref_f32_to_bf16": (u16, [f32]), "ref_bf16_to_f32": (f32, [u16]),
            "ref_f16_to_f32": (f32, [u16]), "ref_f32_to_f16": (u16, [f32]),
            "ref_kv8_f32_to_f16_rne": (u16, [f32]),
            "ref_int4_dequant": (None, [vp, vp, u32, u32, vp]),
            "ref_int4_random": (None, [u32, u32, u32, vp, vp]),
            "ref_repack_layout1": (None, [vp, vp, u32, u32, vp]),
            "ref_interleave16_l0": (None, [vp, vp, vp, vp, u32, u32, vp, vp]),
            "ref_twin_gemv": (None, [u32, vp, vp, u32, u32, vp, u32, u32, vp]),
            "ref_gemv_ref": (None, [u32, vp, vp, u32, u32, vp, u32, vp, vp]),
            "ref_res_norm": (None, [vp, vp, vp, vp, u32, u32, u32]),
            "ref_res_fold": (None, [vp, vp, vp, u32, u32, u32, u32]),
            "ref_norm_finish": (None, [vp, vp, vp, vp, u32, u32, u32]),
            "ref_silu_s": (u32, []),
            "ref_silu_mul": (None, [vp, vp, u32, u32]),
            "ref_attn_prep": (None, [u32, u32, u32, vp, vp, vp, vp, vp, vp, vp]),
            "ref_attn_decode": (None, [u32, u32, u32, u32, vp, vp, vp, vp]),
            "ref_attn_reduce": (None, [u32, u32, u32, u32, vp, vp, vp]),
            "ref_kv8_rotate": (None, [vp, vp]), "ref_kv8_unrotate": (None, [vp, vp]),
            "ref_kv8_encode": (u16, [vp, vp]), "ref_kv8_dequant": (f32, [C.c_int8, u16]),
            "ref_kv8_prep": (None, [u32, u32, u32, vp, vp, vp, u32, vp, vp, vp, vp, vp, vp]),
            "ref_kv8_attend": (None, [vp, u32, vp, vp, vp, vp, u32, u32, vp, vp]),
            "ref_moe_route": (None, [vp, u32, u32, u32, u32, u32, vp]),
            "ref_moe_split_dot": (f32, [vp, u32, u32, vp, u32]),
            "ref_moe_silu_up": (u16, [f32, f32]),
            "ref_moe_combine": (u16, [vp, vp, u32, u32, u16]),
            "ref_moe_block": (None, [vp, u32, u32, u32, u32, u32, vp, vp, vp, u32, u32, vp]),
            "ref_pf_moe_block": (None, [vp, u32, vp, vp, vp, u32, u32, u32, u32, vp]),
            "ref_repack_bf16_tiled": (None, [vp, u32, u32, vp]),
            "ref_quantise_int8_tiled": (None, [vp, u32, u32, vp, vp]),
            "ref_rtn_int4_g64": (None, [vp, u32, u32, vp, vp]),
            "ref_int8_tiled_index": (C.c_size_t, [u32, u32, u32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(R, name)
            fn.restype = res
            fn.argtypes = args
    return _ref


# ---- structures ------------------------------------------------------------------------
class AttnShape(C.Structure):
    _fields_ = [("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("rot_dim", C.c_uint32), ("gated", C.c_uint32), ("qkv_n", C.c_uint32),
                ("k_off", C.c_uint32), ("v_off", C.c_uint32), ("scale", C.c_float),
                ("eps", C.c_float)]


def attn_shape(q_heads, kv_heads, head_dim, rot_dim=None, gated=False, eps=1e-6):
    rot_dim = head_dim if rot_dim is None else rot_dim
    qcols = q_heads * head_dim * (2 if gated else 1)
    k_off = qcols
    v_off = k_off + kv_heads * head_dim
    scale = np.float32(1.0 / np.sqrt(head_dim))
    return AttnShape(q_heads, kv_heads, head_dim, rot_dim, int(gated), v_off + kv_heads * head_dim,
                     k_off, v_off, float(scale), float(eps))


class MoeRoute(C.Structure):
    _fields_ = [("ids", C.c_uint32 * 8), ("w", C.c_float * 8), ("p", C.c_float * 8),
                ("p9", C.c_float), ("sg", C.c_float)]


class Linear(C.Structure):
    _fields_ = [("qweight", C.c_void_p), ("scales", C.c_void_p), ("K", C.c_uint32),
                ("N", C.c_uint32), ("S", C.c_uint32)]


class Layer(C.Structure):
    _fields_ = [("qkv", Linear), ("o", Linear), ("gate_up", Linear), ("down", Linear),
                ("in_norm", C.c_void_p), ("post_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("router", C.c_void_p), ("moe_gu", C.c_void_p),
                ("moe_dn", C.c_void_p)]


class MtpHead(C.Structure):
    """orc_mtp_head: the MTP head's fc, its decoder layer and its three norms."""
    _fields_ = [("fc", Linear), ("layer", Layer), ("pre_e", C.c_void_p), ("pre_h", C.c_void_p),
                ("final_norm", C.c_void_p), ("w16_fc", C.c_void_p), ("w16_qkv", C.c_void_p),
                ("w16_o", C.c_void_p), ("w16_gu", C.c_void_p), ("w16_dn", C.c_void_p)]


class DenseModel(C.Structure):
    _fields_ = [("layers", C.c_uint32), ("hidden", C.c_uint32), ("inter", C.c_uint32),
                ("vocab", C.c_uint32), ("vocab_used", C.c_uint32), ("max_len", C.c_uint32),
                ("attn", AttnShape), ("rms_eps", C.c_float), ("layer", C.c_void_p),
                ("embed", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", Linear),
                ("rope", C.c_void_p), ("tgt", C.c_uint32), ("norm_g", C.c_uint32),
                ("experts", C.c_uint32), ("top_k", C.c_uint32), ("moe_inter", C.c_uint32),
                ("router_n", C.c_uint32), ("router_ksplit", C.c_uint32),
                ("lm_i8", C.c_void_p), ("lm_i8_scales", C.c_void_p)]


# ---- numpy helpers ----------------------------------------------------------------------
def f16_bits_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def widen(act, h):
    return bf16_bits_to_f32(h) if act == ORC_BF16 else f16_bits_to_f32(h)


def f32_to_bf16_bits(f):
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + (((u >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)


def f32_to_f16_bits(f):
    """IEEE RNE (numpy's cast is RNE with subnormals; the oracle's orc_f32_to_f16 agrees)."""
    return np.asarray(f, dtype=np.float32).astype(np.float16).view(np.uint16)


def rne(act, f):
    return f32_to_bf16_bits(f) if act == ORC_BF16 else f32_to_f16_bits(f)


def c32(a):
    return np.ascontiguousarray(a)


# ---- wrappers ----------------------------------------------------------------------------
def int4_dequant(qweight, scales, K, N):
    out = np.empty((K, N), np.float32)
    lib().orc_int4_dequant(_p(c32(qweight)), _p(c32(scales)), K, N, _p(out))
    return out


def gemv_ref(qweight, scales, K, N, xf, layout=0):
    xf = c32(np.asarray(xf, np.float32).reshape(-1, K))
    M = xf.shape[0]
    out = np.empty((M, N), np.float64)
    bound = np.empty((M, N), np.float64)
    lib().orc_gemv_ref(layout, _p(c32(qweight)), _p(scales if scales is None else c32(scales)),
                       K, N, _p(xf), M, _p(out), _p(bound))
    return out, bound


def gemv_twin(qweight, scales, K, N, xf, S=1, layout=0):
    xf = c32(np.asarray(xf, np.float32).reshape(-1, K))
    M = xf.shape[0]
    out = np.empty((M, N), np.float32)
    lib().orc_gemv_twin(layout, _p(c32(qweight)), _p(scales if scales is None else c32(scales)),
                        K, N, _p(xf), M, S, _p(out))
    return out


def n2_over(got, ref, bound):
    got = c32(np.asarray(got, np.float32).ravel())
    ref = c32(np.asarray(ref, np.float64).ravel())
    bound = c32(np.asarray(bound, np.float64).ravel())
    mr = np.zeros(1, np.float64)
    over = lib().orc_n2_over(_p(got), _p(ref), _p(bound), got.size, _p(mr))
    return int(over), float(mr[0])


def res_norm(act, partials, resid, norm_w, M, K, S_PREV, eps=1e-6):
    resid = resid.copy()
    x = np.empty((M, K), np.uint16)
    lib().orc_res_norm(act, _p(partials if partials is None else c32(partials)), _p(resid),
                       _p(c32(norm_w)), _p(x), M, K, S_PREV, eps)
    return resid, x


def silu_mul(act, partials, M, N, S):
    x = np.empty((M, N), np.uint16)
    lib().orc_silu_mul(act, _p(c32(partials)), _p(x), M, N, S)
    return x


def rope_table(theta, rot_dim, max_len):
    t = np.empty((max_len, 2, rot_dim // 2), np.float32)
    lib().orc_rope_table(theta, rot_dim, max_len, _p(t))
    return t


def argmax(logits, vocab_used=None):
    logits = c32(np.asarray(logits, np.float32))
    return int(lib().orc_argmax(_p(logits), logits.size,
                                logits.size if vocab_used is None else vocab_used))


def accept_greedy(verify_argmax, drafts):
    va = c32(np.asarray(verify_argmax, np.uint32))
    dr = c32(np.asarray(drafts, np.uint32))
    nxt = np.zeros(1, np.uint32)
    j = lib().orc_accept_greedy(_p(va), _p(dr), dr.size, _p(nxt))
    return int(j), int(nxt[0])
