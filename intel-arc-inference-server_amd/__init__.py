"""MI355X-native decode loop - host-side Python binding of libmi355x_decode.so.

The product is the HIP library and its C ABI (include/mi355x_decode.h); this module
only loads it with ctypes and declares the signatures. There is no fallback: if the
library is missing, loading fails with an error naming the build step.
"""
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.environ.get("MI355X_DECODE_LIB") or os.path.join(HERE, "libmi355x_decode.so")
HEADER = os.path.join(ROOT, "include", "mi355x_decode.h")

_lib = None

u8, u16, u32, u64, i32, f32, sz, vp = (C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int,
                                        C.c_float, C.c_size_t, C.c_void_p)

# name -> (restype, argtypes)
SIGNATURES = {
    "mi_last_error": (C.c_char_p, []),
    "mi_malloc": (i32, [C.POINTER(vp), sz]),
    "mi_free": (i32, [vp]),
    "mi_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "mi_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "mi_memcpy_d2d": (i32, [vp, vp, sz, vp]),
    "mi_stream_sync": (i32, [vp]),
    "mi_device_sync": (i32, []),
    "mi_event_create": (i32, [C.POINTER(vp)]),
    "mi_event_record": (i32, [vp, vp]),
    "mi_event_elapsed_ms": (i32, [vp, vp, C.POINTER(f32)]),
    "mi_event_destroy": (i32, [vp]),
    "mi_fill_u32": (i32, [vp, sz, u64, vp]),
    "mi_fill_f16": (i32, [vp, sz, u64, i32, f32, f32, vp]),
    "mi_fill_f32": (i32, [vp, sz, u64, i32, f32, f32, i32, vp]),
    "mi_fill_layout1": (i32, [vp, sz, u64, f32, f32, vp]),
    "mi_f16_to_bf16": (i32, [vp, sz, u32, vp]),
    "mi_fill_i8": (i32, [vp, sz, u64, i32, i32, vp]),
    "mi_int4_dequant": (i32, [vp, vp, vp, u32, u32, vp]),
    "mi_gemv_w4a16": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_gemv_pick_s": (u32, [u32, u32]),
    "mi_gemv_pick_s_ex": (u32, [u32, u32, u32]),
    "mi_fold_partials": (i32, [vp, vp, vp, u32, u32, u32, vp]),
    "mi_gemv_handoff_init": (i32, [vp, sz, vp]),
    "mi_stream_read": (i32, [vp, sz, vp, vp]),
    "mi_res_fold": (i32, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_norm_finish": (i32, [vp, vp, vp, vp, u32, u32, u32, f32, vp]),
    "mi_res_norm": (i32, [vp, vp, vp, vp, u32, u32, u32, f32, vp]),
    "mi_silu_mul": (i32, [vp, vp, u32, u32, u32, vp]),
    "mi_attn_prep": (i32, [vp, vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, vp, u32, u32, vp]),
    "mi_attn_prep_kv8": (i32, [vp, vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, vp, u32,
                               u32, vp]),
    "mi_attn_ppw": (u32, [u32, u32]),
    "mi_attn_verify": (i32, [vp, vp, vp, vp, sz, sz, vp, u32, u32, vp, u32, u32, vp, vp]),
    "mi_attn_verify_binds": (i32, [u32, u32, u32, u32]),
    "mi_attn_decode": (i32, [vp, vp, u32, vp, vp, vp, vp, sz, sz, sz, sz, vp, u32, u32, vp, u32, u32, vp, vp]),
    "mi_attn_reduce": (i32, [vp, vp, vp, vp, u32, u32, u32, vp, vp]),
    "mi_attn_prep_decode": (i32, [vp, vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, sz, sz, vp, u32, u32, vp, u32, vp]),
    "mi_attn_reduce_kv8": (i32, [vp, vp, vp, vp, u32, u32, u32, vp, vp]),
    "mi_embed_gather": (i32, [vp, vp, vp, u32, u32, u32, vp]),
    "mi_argmax_groups": (u32, [u32]),
    "mi_argmax": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_argmax_static": (i32, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_argmax_finish": (i32, [vp, vp, u32, vp, u32, vp]),
    "mi_embed_norm": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, u32, f32, vp]),
    "mi_embed_norm_act": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, u32, f32, u32, vp]),
    "mi_gemv_w4a16_ex": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp, vp]),
    "mi_engine_create": (vp, [vp, u64, vp]),
    "mi_checkpoint_desc": (i32, [C.c_char_p, u32, u32, vp]),
    "mi_engine_load": (i32, [vp, C.c_char_p, C.c_char_p, sz]),
    "mi_checkpoint_check": (i32, [C.c_char_p, C.c_char_p, sz]),
    "mi_engine_destroy": (None, [vp]),
    "mi_engine_stream": (vp, [vp]),
    "mi_engine_tensor": (i32, [vp, u32, u32, C.POINTER(vp), C.POINTER(sz)]),
    "mi_engine_linear_s": (i32, [vp, u32, C.POINTER(u32)]),
    "mi_engine_capture": (i32, [vp, u32]),
    "mi_engine_reset": (i32, [vp, u32, u32]),
    "mi_engine_replay": (i32, [vp, u32]),
    "mi_engine_step_eager": (i32, [vp, u32]),
    "mi_engine_generate": (i32, [vp, u32, vp]),
    "mi_engine_ingest": (i32, [vp, vp, u32]),
    "mi_engine_prefill": (i32, [vp, vp, u32, u32]),
    "mi_gemm_w4a16": (i32, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "mi_gemm_w4a16_silu": (i32, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "mi_attn_prefill": (i32, [vp, vp, vp, sz, sz, vp, u32, u32, u32, vp, vp, vp]),
    "mi_embed_rows": (i32, [vp, vp, vp, u32, u32, u32, vp, vp]),
    "mi_moe_prefill": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, vp, vp, vp, vp, vp, vp]),
    "mi_attn_prep_rows": (i32, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, sz, sz, vp, u32, vp]),
    "mi_attn_prefill_kv8": (i32, [vp, vp, vp, vp, vp, sz, sz, sz, sz, vp, u32, u32, u32, vp, vp, vp, vp]),
    "mi_engine_bench_linear": (i32, [vp, u32, u32, vp]),
    "mi_engine_bench_verify": (i32, [vp, u32, u32, vp]),
    "mi_engine_read_ctrl": (i32, [vp, vp]),
    "mi_engine_verify": (i32, [vp, vp, u32, vp]),
    "mi_engine_commit": (i32, [vp, u32, u32, u32]),
    "mi_engine_draft": (i32, [vp, u32, vp]),
    "mi_i8w_index": (sz, [u32, u32, u32]),
    "mi_lm_head_int8_quantise": (i32, [vp, u32, u32, vp, vp]),
    "mi_i8w_from_ref_tiles": (i32, [vp, u32, u32, vp, vp]),
    "mi_gemv_i8w": (i32, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "mi_res_fold_ex": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "mi_norm_finish_ex": (i32, [vp, vp, vp, vp, sz, u32, u32, u32, f32, vp]),
    "mi_accept_greedy": (u32, [vp, vp, u32, vp]),
    "mi_norm_rows": (i32, [vp, vp, vp, vp, u32, u32, f32, vp]),
    "mi_gemv_f16w": (i32, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_moe_route": (i32, [vp, vp, u32, u32, u32, u32, vp]),
    "mi_moe_gate_up": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "mi_moe_gate_up_routed": (i32, [vp, u32, vp, vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "mi_moe_down_norm": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp, vp, vp, f32, vp, vp, u32, u32, vp]),
    "mi_moe_down": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp]),
}


EPI_PARTIALS, EPI_RESID, EPI_SILU, EPI_LOGITS, EPI_F16OUT, EPI_QKV = 0, 1, 2, 3, 4, 5


class GemvEpilogue(C.Structure):
    """mi_gemv_epilogue"""
    _fields_ = [("kind", u32), ("resid", vp), ("sumsq", vp), ("rstd", vp),
                ("next_norm_w", vp), ("x_next", vp), ("eps", f32), ("h", vp), ("logits", vp),
                ("argmax_part", vp), ("vocab_used", u32), ("out16", vp),
                ("ctrl", vp), ("shape", vp), ("q_norm", vp), ("k_norm", vp), ("rope", vp), ("attn_q", vp),
                ("kv_k", vp), ("kv_v", vp), ("row_stride", sz), ("head_stride", sz), ("pages", vp),
                ("page", u32), ("kv_len", u32), ("status", vp), ("poll_limit", u32), ("inject", u32),
                ("arrive", vp), ("act", u32), ("sums_out", vp), ("in_sums", vp), ("in_norm_w", vp),
                ("in_eps", f32)]


STATUS_HANDOFF_TIMEOUT = 0xDEAD0003


class MiError(RuntimeError):
    pass


def lib():
    """The loaded library (raises MiError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MiError(f"{LIB_PATH} is missing: run `python __graft_entry__.py` (build()) first")
        # One HIP runtime per process: PyTorch ships its own libamdhip64 under the same soname,
        # and the one loaded first serves both. Loading torch first makes that its runtime, so
        # torch tensors (device buffers, streams) work whatever this library is called with.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, what=""):
    """Raise MiError on a non-zero return code, with the library's message."""
    if rc != 0:
        msg = lib().mi_last_error().decode(errors="replace")
        raise MiError(f"{what or 'call'} failed ({rc}): {msg}")
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args), name)


def header_functions():
    """Every function the public header declares (for the export check)."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


class AttnShape(C.Structure):
    """mi_attn_shape: heads, head_dim, rotary dims, gate on/off, the fused qkv column map."""
    _fields_ = [("q_heads", u32), ("kv_heads", u32), ("head_dim", u32), ("rot_dim", u32),
                ("gated", u32), ("qkv_n", u32), ("k_off", u32), ("v_off", u32), ("scale", f32),
                ("eps", f32), ("act", u32)]


def lib_shape(sh, act=0):
    """An mi_attn_shape with the fields of `sh` (this package's AttnShape or the oracle's
    orc_attn_shape, which has the same leading fields) and the activation type act."""
    names = [f[0] for f in AttnShape._fields_ if f[0] != "act"]
    return AttnShape(*[getattr(sh, n) for n in names], act)


def shape_ref(sh, act=0):
    """A pointer to lib_shape(sh, act), for the entries that take `const mi_attn_shape*`."""
    return C.byref(lib_shape(sh, act))


# ---- the decode loop (host-side mirror of src/runtime/engine.h) -------------------------
class ModelDesc(C.Structure):
    """mi_model_desc: the model's shape as data (model::ModelDesc)."""
    _fields_ = [("layers", u32), ("hidden", u32), ("q_heads", u32), ("kv_heads", u32),
                ("head_dim", u32), ("rot_dim", u32), ("inter", u32), ("vocab", u32),
                ("vocab_used", u32), ("max_len", u32), ("qk_norm", u32), ("max_rows", u32),
                ("attn_tgt", u32), ("rope_theta", f32), ("rms_eps", f32),
                ("experts", u32), ("top_k", u32), ("moe_inter", u32), ("kv_int8", u32),
                ("mtp", u32), ("lm_head_int8", u32), ("act_bf16", u32), ("mtp_w16", u32)]


def dense_desc(layers, hidden, q_heads, kv_heads, head_dim, inter, vocab, max_len, *,
               rot_dim=None, vocab_used=None, qk_norm=1, max_rows=8, attn_tgt=128,
               rope_theta=1e6, rms_eps=1e-6, kv_int8=0, mtp=0, lm_head_int8=0, act_bf16=0, mtp_w16=0):
    d = ModelDesc(layers, hidden, q_heads, kv_heads, head_dim,
                  head_dim if rot_dim is None else rot_dim, inter, vocab,
                  vocab if vocab_used is None else vocab_used, max_len, qk_norm, max_rows,
                  attn_tgt, rope_theta, rms_eps)
    d.kv_int8 = kv_int8
    d.mtp = mtp
    d.lm_head_int8 = lm_head_int8
    d.act_bf16 = act_bf16
    d.mtp_w16 = mtp_w16
    return d


def moe_desc(layers, hidden, q_heads, kv_heads, head_dim, experts, top_k, moe_inter, vocab, max_len,
             **kw):
    """A mixture-of-experts decoder: every layer is attention + the MoE block (experts routed,
    top_k per token, one shared expert, expert intermediate moe_inter)."""
    d = dense_desc(layers, hidden, q_heads, kv_heads, head_dim, 0, vocab, max_len, **kw)
    d.experts, d.top_k, d.moe_inter = experts, top_k, moe_inter
    return d


def checkpoint_check(ckpt_dir):
    """mi_checkpoint_check: the quantisation checks of a checkpoint directory; its report."""
    buf = C.create_string_buffer(512)
    check(lib().mi_checkpoint_check(os.fsencode(ckpt_dir), buf, len(buf)), "checkpoint_check")
    return buf.value.decode()


def checkpoint_desc(ckpt_dir, max_len, max_rows=8):
    """mi_checkpoint_desc: the model description a checkpoint's config.json gives."""
    d = ModelDesc()
    check(lib().mi_checkpoint_desc(os.fsencode(ckpt_dir), max_len, max_rows, C.byref(d)), "checkpoint_desc")
    return d


def desc_moe_cfg4(max_len=4096 + 512):
    """a 40-layer MoE decoder, hidden 2048, 256 experts top 8 + 1 shared,
    expert intermediate 512, attention 16 q / 2 kv heads of 256, vocab 151936 (assumed; the
    config does not state it), RoPE theta 1e6. Attention blocks per kv head: 64 (at context 4096,
    blocks of 128 positions: 2 x 33 work-groups; the step measured 2.445 ms against 2.51 at 128
    blocks of 64 positions, whose merge reads twice the partials)."""
    return moe_desc(40, 2048, 16, 2, 256, 256, 8, 512, 151936, max_len, attn_tgt=64)


def desc_27b(max_len=4096 + 512, act_bf16=0):
    """the 27B-shape dense decoder (64 layers, hidden 5120, 40 q / 8 kv
    heads of 128, SwiGLU 17408, vocab 151936, RoPE theta 1e6). Attention blocks per kv head:
    64 (at context 4096, blocks of 128 positions: 8 x 33 work-groups, measured faster than
    128 blocks of 64 positions)."""
    return dense_desc(64, 5120, 40, 8, 128, 17408, 151936, max_len, attn_tgt=64, act_bf16=act_bf16)


# tensor kinds (mi_engine_tensor)
(T_QKV_Q, T_QKV_S, T_O_Q, T_O_S, T_GU_Q, T_GU_S, T_DOWN_Q, T_DOWN_S, T_IN_NORM, T_POST_NORM,
 T_Q_NORM, T_K_NORM, T_ROUTER, T_MOE_GU, T_MOE_DN) = range(15)
(T_EMBED, T_FINAL_NORM, T_LM_Q, T_LM_S, T_ROPE, T_KV_K, T_KV_V, T_LOGITS, T_CTRL,
 T_HISTORY, T_KV_KS, T_KV_VS, T_RESID, T_X, T_ATTN_Q, T_ATTN_OUT, T_HBUF, T_MTP_FC_Q, T_MTP_FC_S,
 T_MTP_PRE_E, T_MTP_PRE_H, T_MTP_FINAL, T_MTP_KV_K, T_MTP_KV_V, T_MTP_HH, T_MTP_DH, T_MTP_CTRL, T_MTP_LOGITS,
 T_LM_I8, T_LM_I8_S, T_MOE_HANDOFF, T_MTP_W16_FC, T_MTP_W16_QKV, T_MTP_W16_O, T_MTP_W16_GU,
 T_MTP_W16_DN) = range(32, 68)
CTRL_POS, CTRL_NACT, CTRL_CUR, CTRL_OUT, CTRL_DEBUG, CTRL_STEPS, CTRL_WORDS = 0, 1, 2, 10, 18, 19, 192
CTRL_WIDE_CUR, CTRL_WIDE_OUT, CTRL_DEEP_CUR, CTRL_DEEP_OUT = 32, 48, 64, 128


class Engine:
    """Owns a mi_engine: weights, KV cache, the captured step graphs."""

    def __init__(self, desc, seed=1234, stream=None):
        self.desc = desc
        self._h = lib().mi_engine_create(C.byref(desc), seed, stream)
        if not self._h:
            raise MiError("mi_engine_create: " + lib().mi_last_error().decode(errors="replace"))

    def close(self):
        if self._h:
            lib().mi_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return lib().mi_engine_stream(self._h)

    def load(self, ckpt_dir):
        """mi_engine_load: a GPTQ / AutoRound int4 g64 checkpoint directory; returns the
        loader's one-line report."""
        buf = C.create_string_buffer(512)
        check(lib().mi_engine_load(self._h, os.fsencode(ckpt_dir), buf, len(buf)), "engine_load")
        return buf.value.decode()

    def tensor(self, kind, layer=0):
        p, b = vp(), sz()
        check(lib().mi_engine_tensor(self._h, kind, layer, C.byref(p), C.byref(b)), "engine_tensor")
        return p.value, b.value

    def to_host(self, kind, layer=0, dtype="uint8"):
        import numpy as np
        p, b = self.tensor(kind, layer)
        out = np.empty(b, np.uint8)
        if b:
            check(lib().mi_memcpy_d2h(out.ctypes.data, p, b, self.stream), "d2h")
        return out.view(dtype)

    def from_host(self, kind, arr, layer=0):
        import numpy as np
        p, b = self.tensor(kind, layer)
        a = np.ascontiguousarray(arr)
        assert a.nbytes == b, (a.nbytes, b)
        check(lib().mi_memcpy_h2d(p, a.ctypes.data, b, self.stream), "h2d")
        check(lib().mi_stream_sync(self.stream), "sync")

    def linear_s(self, which):
        s = u32()
        check(lib().mi_engine_linear_s(self._h, which, C.byref(s)), "linear_s")
        return s.value

    def capture(self, M=1):
        check(lib().mi_engine_capture(self._h, M), "engine_capture")

    def reset(self, pos, token):
        check(lib().mi_engine_reset(self._h, pos, token), "engine_reset")

    def replay(self, M=1):
        check(lib().mi_engine_replay(self._h, M), "engine_replay")

    def step_eager(self, M=1):
        check(lib().mi_engine_step_eager(self._h, M), "engine_step_eager")

    def generate(self, n):
        import numpy as np
        out = np.zeros(n, np.uint32)
        check(lib().mi_engine_generate(self._h, n, out.ctypes.data), "engine_generate")
        return out

    def ingest(self, ids):
        import numpy as np
        a = np.ascontiguousarray(ids, np.uint32)
        check(lib().mi_engine_ingest(self._h, a.ctypes.data, a.size), "engine_ingest")

    def prefill(self, ids, chunk=0):
        """Engine::prefill: the ids in chunks of at most `chunk` positions (0: the cap)."""
        import numpy as np
        a = np.ascontiguousarray(ids, np.uint32)
        check(lib().mi_engine_prefill(self._h, a.ctypes.data, a.size, chunk), "engine_prefill")

    def ctrl(self):
        import numpy as np
        out = np.zeros(CTRL_WORDS, np.uint32)
        check(lib().mi_engine_read_ctrl(self._h, out.ctypes.data), "engine_read_ctrl")
        return out

    def verify(self, drafts):
        import numpy as np
        d = np.ascontiguousarray(drafts, np.uint32)
        out = np.zeros(d.size + 1, np.uint32)
        check(lib().mi_engine_verify(self._h, d.ctypes.data if d.size else None, d.size, out.ctypes.data),
              "engine_verify")
        return out

    def commit(self, verify_pos, j, nxt):
        check(lib().mi_engine_commit(self._h, verify_pos, j, nxt), "engine_commit")

    def draft(self, k):
        """Engine::draft: k greedy drafts from the MTP head (mtp models)."""
        import numpy as np
        out = np.zeros(k, np.uint32)
        check(lib().mi_engine_draft(self._h, k, out.ctypes.data), "engine_draft")
        return out

    def logits(self, rows=1):
        import numpy as np
        lg = self.to_host(T_LOGITS, dtype=np.float32)
        return lg[:rows * self.desc.vocab].reshape(rows, self.desc.vocab)


def accept_greedy(verify_argmax, drafts):
    """server::accept_greedy through the library: (accepted count j, next token)."""
    import numpy as np
    va = np.ascontiguousarray(verify_argmax, np.uint32)
    d = np.ascontiguousarray(drafts, np.uint32)
    nxt = u32()
    j = lib().mi_accept_greedy(va.ctypes.data, d.ctypes.data if d.size else None, d.size, C.byref(nxt))
    return int(j), int(nxt.value)
