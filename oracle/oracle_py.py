"""ctypes binding of liboracle.so - TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by
the product. The oracle restates the reference verify path on the CPU (see
oracle.cpp for the reference lines each function follows).
"""
import ctypes
import os
import sys
from ctypes import POINTER, c_float, c_int32, c_int64, c_uint16, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "moss-transcribe.cpp_amd"))
import mtg  # noqa: E402  (struct definitions shared with the C ABI)


class Target(ctypes.Structure):
    pass


VERIFY_FN = ctypes.CFUNCTYPE(c_int32, POINTER(Target), POINTER(c_int32), c_int32, POINTER(c_int32),
                             c_int32, c_float, POINTER(c_int32), POINTER(c_int32))
Target._fields_ = [("self", c_void_p), ("verify", VERIFY_FN), ("past", c_int32),
                   ("max_seq", c_int32), ("vocab", c_int32)]

SIGNATURES = {
    "orc_create": (c_int32, [POINTER(mtg.ModelDesc), c_int32, c_int32, POINTER(c_void_p)]),
    "orc_destroy": (None, [c_void_p]),
    "orc_past_len": (c_int32, [c_void_p]),
    "orc_rewind": (c_int32, [c_void_p, c_int32]),
    "orc_set_threads": (None, [c_int32]),
    "orc_embed": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "orc_run": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "orc_prefill": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "orc_logits": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "orc_verify": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_float, c_void_p,
                             c_void_p, c_void_p, c_void_p]),
    "orc_kv_write": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32]),
    "orc_kv_read": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32]),
    "orc_ngram_draft": (c_int32, [c_void_p, c_int32, c_int32, c_void_p]),
    "orc_greedy_choice": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_float]),
    "orc_controller": (c_int32, [POINTER(Target), c_int32, c_void_p, c_int32, c_int32, c_int32,
                                 c_int32, c_float, c_int32, c_void_p, c_void_p, c_void_p,
                                 POINTER(c_int32), POINTER(mtg.GenStats)]),
    "orc_generate_from": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                    c_float, c_int32, c_void_p, c_void_p, c_void_p,
                                    POINTER(c_int32), POINTER(mtg.GenStats)]),
    "orc_f32_to_f16": (c_uint16, [c_float]),
    "orc_exp": (c_float, [c_float]),
    "orc_f16_to_f32": (c_float, [c_uint16]),
    "orc_quantize_q8_0_act": (None, [c_void_p, c_int64, c_void_p]),
    "orc_quantize_q8_k_act": (None, [c_void_p, c_int64, c_void_p]),
    "orc_set_order": (c_int32, [c_void_p, c_int32]),
    "orc_mul_mat_generic": (None, [c_int32, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "orc_q8_0_block_dot": (c_int32, [c_void_p, c_void_p]),
    "orc_q8_0_block_dots": (None, [c_void_p, c_void_p, c_int32, c_void_p]),
    "orc_mul_mat": (None, [c_int32, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "orc_rms_norm": (None, [c_void_p, c_void_p, c_int32, c_float, c_void_p]),
    "orc_rope_neox": (None, [c_void_p, c_int32, c_int32, c_float]),
    "orc_softmax": (None, [c_void_p, c_int32, c_float, c_void_p, c_void_p]),
    "orc_causal_context": (None, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                  c_void_p]),
    "orc_attention": (None, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                             c_void_p, c_void_p]),
    "orc_encoder_create": (c_int32, [POINTER(mtg.EncoderDesc), POINTER(c_void_p)]),
    "orc_encoder_destroy": (None, [c_void_p]),
    "orc_encoder_encode": (c_int32, [c_void_p, c_void_p, c_void_p, POINTER(c_int32)]),
    "orc_encoder_adapt": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, POINTER(c_int32)]),
    "orc_gelu_erf": (c_float, [c_float]),
    "orc_layer_norm": (None, [c_void_p, c_void_p, c_void_p, c_int32, c_float, c_void_p]),
    "orc_conv1d": (None, [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_int32, c_void_p]),
    "orc_enc_attention": (None, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError("liboracle.so is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


ptr = mtg.ptr
i32 = mtg.i32
f32 = mtg.f32

Q8_BLOCK = np.dtype([("d", "<u2"), ("qs", "i1", 32)])


def quantize_q8_0_act(x):
    x = f32(x)
    out = np.zeros(x.size // 32, Q8_BLOCK)
    lib().orc_quantize_q8_0_act(ptr(x), x.size, ptr(out))
    return out


Q8K_BLOCK = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])


def quantize_q8_k_act(x):
    x = f32(x)
    out = np.zeros(x.size // 256, Q8K_BLOCK)
    assert out.itemsize == 4 + 256 + 32
    lib().orc_quantize_q8_k_act(ptr(x), x.size, ptr(out))
    return out


def mul_mat(wtype, w_bytes, k, n, x):
    x = f32(x)
    T = x.shape[0]
    y = np.empty((T, n), np.float32)
    lib().orc_mul_mat(wtype, ptr(w_bytes), k, n, ptr(x), T, ptr(y))
    return y


def mul_mat_generic(wtype, w_bytes, k, n, x):
    """mul_mat in ggml's generic scalar order (sequential block sums)."""
    x = f32(x)
    T = x.shape[0]
    y = np.empty((T, n), np.float32)
    lib().orc_mul_mat_generic(wtype, ptr(w_bytes), k, n, ptr(x), T, ptr(y))
    return y


def rms_norm(x, w, eps):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rms_norm(ptr(x), ptr(w), x.size, eps, ptr(y))
    return y


def rope_neox(x, pos, base):
    x = f32(x).copy()
    lib().orc_rope_neox(ptr(x), x.size, pos, base)
    return x


def softmax(s, scale, mask=None):
    s = f32(s)
    out = np.empty_like(s)
    m = f32(mask) if mask is not None else None
    lib().orc_softmax(ptr(s), s.size, scale, ptr(m), ptr(out))
    return out


def causal_context(v, p, kv_heads, heads, queries, kv_len, head_dim):
    v, p = f32(v), f32(p)
    out = np.empty((heads, queries, head_dim), np.float32)
    lib().orc_causal_context(ptr(v), ptr(p), head_dim, kv_heads, heads, queries, kv_len, ptr(out))
    return out


def attention(q, k, v, past):
    """The decoder step's canonical attention: q [T][heads][head_dim] (float32),
    k, v [kv_heads][max_seq][head_dim] float32 or float16 holding keys
    [0, past + T). Returns [T][heads][head_dim]."""
    q = f32(q)
    T, heads, hd = q.shape
    f16kv = k.dtype == np.float16
    k, v = np.ascontiguousarray(k), np.ascontiguousarray(v)
    assert k.dtype == v.dtype and k.shape == v.shape and k.shape[1] >= past + T
    out = np.empty((T, heads, hd), np.float32)
    lib().orc_attention(ptr(k), ptr(v), int(f16kv), k.shape[1], past, T, heads, k.shape[0], hd, ptr(q), ptr(out))
    return out


def ngram_draft(history, maximum):
    h = i32(history)
    out = np.zeros(max(maximum, 1), np.int32)
    n = lib().orc_ngram_draft(ptr(h) if len(h) else None, len(h), maximum, ptr(out))
    return [int(x) for x in out[:n]]


def greedy_choice(raw, history, penalty):
    raw = f32(raw)
    h = i32(history)
    return int(lib().orc_greedy_choice(ptr(raw), len(raw), ptr(h) if len(h) else None, len(h),
                                       penalty))


def run_controller(verify_cb, first_seed, max_new, eos, penalty=1.0, max_draft=4, past=0,
                   max_seq=1 << 20, vocab=1 << 20, draft=None, max_steps=0):
    """Drive orc_controller with a Python target: verify_cb(tokens, history, penalty)
    returns (choices, n_match)."""
    def _verify(tg, tokens, T, hist, nh, pen, choice_out, n_match_out):
        toks = [tokens[i] for i in range(T)]
        h = [hist[i] for i in range(nh)]
        ch, nm = verify_cb(toks, h, pen, tg.contents.past)
        for i in range(T):
            choice_out[i] = int(ch[i])
        n_match_out[0] = int(nm)
        return 0
    cb = VERIFY_FN(_verify)
    tg = Target(None, cb, past, max_seq, vocab)
    out = np.empty(max_new, np.int32)
    n = c_int32(0)
    st = mtg.GenStats()
    keep = None
    fn = None
    if draft is not None:
        def _d(_u, ids, n_ids, budget, dst):
            props = list(draft([ids[i] for i in range(n_ids)], budget))[:budget]
            for i, t in enumerate(props):
                dst[i] = int(t)
            return len(props)
        keep = mtg.DRAFT_FN(_d)
        fn = ctypes.cast(keep, c_void_p)
    rc = lib().orc_controller(ctypes.byref(tg), first_seed, None, 0, max_new, max_steps, eos, penalty,
                              max_draft, fn, None, ptr(out), ctypes.byref(n), ctypes.byref(st))
    del keep
    if rc:
        raise RuntimeError("orc_controller failed: %d" % rc)
    return [int(x) for x in out[: n.value]], st, tg.past


class Oracle:
    """CPU decoder state (orc_model) over a SynthModel's host tensors."""

    def __init__(self, model, max_seq, kv_type=mtg.TYPE_F32):
        # a copy: a parsed file's hyper-parameters live in the file handle's memory
        self.hp = mtg.Hparams()
        ctypes.memmove(ctypes.byref(self.hp), ctypes.byref(model.hp), ctypes.sizeof(mtg.Hparams))
        self.kv_type = kv_type
        out = c_void_p()
        rc = lib().orc_create(model.desc, max_seq, kv_type, ctypes.byref(out))
        if rc:
            raise RuntimeError("orc_create failed: %d" % rc)
        self.m = out

    ORDER_CANONICAL, ORDER_GGML_GENERIC = 0, 1

    def set_order(self, order):
        """Float order of the step's reductions: ORDER_CANONICAL (the device's) or
        ORDER_GGML_GENERIC (ggml's generic scalar kernels)."""
        rc = lib().orc_set_order(self.m, order)
        if rc:
            raise RuntimeError("orc_set_order %d" % rc)

    def close(self):
        if self.m:
            lib().orc_destroy(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def past_len(self):
        return lib().orc_past_len(self.m)

    def rewind(self, pos):
        rc = lib().orc_rewind(self.m, pos)
        if rc:
            raise RuntimeError("rewind %d" % rc)

    def embed(self, ids):
        ids = i32(ids)
        out = np.empty((len(ids), self.hp.hidden), np.float32)
        assert lib().orc_embed(self.m, ptr(ids), len(ids), ptr(out)) == 0
        return out

    def run(self, embeds):
        embeds = f32(embeds)
        T = embeds.shape[0]
        hid = np.empty((T, self.hp.hidden), np.float32)
        rc = lib().orc_run(self.m, ptr(embeds), T, ptr(hid))
        if rc:
            raise RuntimeError("orc_run %d" % rc)
        return hid

    def prefill(self, embeds):
        embeds = f32(embeds)
        S = embeds.shape[0]
        hid = np.empty((S, self.hp.hidden), np.float32)
        assert lib().orc_prefill(self.m, ptr(embeds), S, ptr(hid)) == 0
        return hid

    def logits(self, hidden):
        hidden = f32(hidden)
        out = np.empty((hidden.shape[0], self.hp.vocab), np.float32)
        assert lib().orc_logits(self.m, ptr(hidden), hidden.shape[0], ptr(out)) == 0
        return out

    def verify(self, tokens, history=(), penalty=1.0, want_hidden=False, want_logits=False):
        tokens = i32(tokens)
        T = len(tokens)
        hist = i32(history)
        choice = np.empty(T, np.int32)
        n_match = np.zeros(1, np.int32)
        hid = np.empty((T, self.hp.hidden), np.float32) if want_hidden else None
        lg = np.empty((T, self.hp.vocab), np.float32) if want_logits else None
        rc = lib().orc_verify(self.m, ptr(tokens), T, ptr(hist) if len(hist) else None, len(hist),
                              penalty, ptr(choice), ptr(n_match), ptr(hid), ptr(lg))
        if rc:
            raise RuntimeError("orc_verify %d" % rc)
        return choice, int(n_match[0]), hid, lg

    def kv_dtype(self):
        return np.float32 if self.kv_type == mtg.TYPE_F32 else np.float16

    def kv_read(self, n_pos):
        shape = (self.hp.n_layers, self.hp.n_kv_heads, n_pos, self.hp.head_dim)
        k = np.empty(shape, self.kv_dtype())
        v = np.empty(shape, self.kv_dtype())
        assert lib().orc_kv_read(self.m, ptr(k), ptr(v), n_pos) == 0
        return k, v

    def kv_write(self, k, v):
        k = np.ascontiguousarray(k, self.kv_dtype())
        v = np.ascontiguousarray(v, self.kv_dtype())
        assert lib().orc_kv_write(self.m, ptr(k), ptr(v), k.shape[2]) == 0

    def generate_from(self, first_seed, max_new, max_steps=0, eos=-1, penalty=1.0, max_draft=4,
                      draft=None, user=None, prior=()):
        out = np.empty(max_new, np.int32)
        n = c_int32(0)
        st = mtg.GenStats()
        prior = i32(prior)
        rc = lib().orc_generate_from(self.m, first_seed, ptr(prior) if len(prior) else None,
                                     len(prior), max_new, max_steps, eos, penalty, max_draft, draft,
                                     user, ptr(out), ctypes.byref(n), ctypes.byref(st))
        if rc:
            raise RuntimeError("orc_generate_from %d" % rc)
        return out[: n.value].copy(), st


class OracleEncoder:
    """CPU restatement of the Whisper encoder + adaptor (orc_encoder_*)."""

    def __init__(self, synth):
        # a copy: synth.hp may be a view into memory its owner frees (a GGUF file's
        # description is released by mtg_gguf_close)
        self.hp = mtg.EncoderHparams()
        ctypes.memmove(ctypes.byref(self.hp), ctypes.byref(synth.hp), ctypes.sizeof(mtg.EncoderHparams))
        self.rows = synth.rows
        out = c_void_p()
        rc = lib().orc_encoder_create(ctypes.byref(synth.desc), ctypes.byref(out))
        if rc:
            raise RuntimeError("orc_encoder_create %d" % rc)
        self.h = out

    def encode(self, mel):
        mel = np.ascontiguousarray(mel, np.float32)
        out = np.empty((self.rows, self.hp.d_model), np.float32)
        n = c_int32(0)
        assert lib().orc_encoder_encode(self.h, ptr(mel), ptr(out), ctypes.byref(n)) == 0
        return out

    def adapt(self, T, rows=None):
        out = np.empty((max(1, T // self.hp.merge), self.hp.hidden), np.float32)
        n = c_int32(0)
        r = None if rows is None else np.ascontiguousarray(rows, np.float32)
        assert lib().orc_encoder_adapt(self.h, ptr(r), T, ptr(out), ctypes.byref(n)) == 0
        return out[: n.value]

    def close(self):
        if self.h:
            lib().orc_encoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gelu_erf(x):
    return float(lib().orc_gelu_erf(float(x)))


def layer_norm(x, w, b, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_layer_norm(ptr(x), ptr(np.ascontiguousarray(w, np.float32)), ptr(np.ascontiguousarray(b, np.float32)),
                         x.size, eps, ptr(y))
    return y


def conv1d(w, x, stride):
    """w [oc][ic][3], x [ic][L] -> [OL][oc]"""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    oc, ic, _ = w.shape
    L = x.shape[1]
    y = np.empty(((L - 1) // stride + 1, oc), np.float32)
    lib().orc_conv1d(ptr(w), ic, oc, ptr(x), L, stride, ptr(y))
    return y


def enc_attention(q, k, v, n_heads):
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    T, W = q.shape
    out = np.empty_like(q)
    lib().orc_enc_attention(ptr(q), ptr(k), ptr(v), T, n_heads, W // n_heads, ptr(out))
    return out
