"""ctypes binding of libmtg.so (include/mtg_verify.h).

The Python layer is plumbing for tests and the benchmark: it passes host numpy
arrays (and, for the *_dev entry points, device pointers from torch tensors) to
the C ABI. The product path is the C++/HIP library; this module raises if it is
missing instead of falling back to anything.
"""
import ctypes
import os
from ctypes import POINTER, c_float, c_int32, c_int64, c_uint16, c_uint64, c_void_p, c_double

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmtg.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K = 0, 1, 8, 12
EXEC_STEP_KERNEL, EXEC_GRAPH, EXEC_EAGER = 0, 1, 2
PROFILE_SLOTS = 9216  # MTG_PROFILE_SLOTS
MAX_BATCH = 16
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_DEVICE, ERR_CAPACITY, ERR_NOMEM, ERR_STATE = 0, -1, -2, -3, -4, -5, -6

QWEN3_0_6B = dict(hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
                  n_layers=28, vocab=151936, rope_base=1e6, rms_eps=1e-6)


class Hparams(ctypes.Structure):
    _fields_ = [("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
                ("head_dim", c_int32), ("intermediate", c_int32), ("n_layers", c_int32),
                ("vocab", c_int32), ("rope_base", c_float), ("rms_eps", c_float)]


class LayerTensors(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_o",
                                        "attn_q_norm", "attn_k_norm", "ffn_norm", "ffn_gate",
                                        "ffn_up", "ffn_down")]


class ModelDesc(ctypes.Structure):
    _fields_ = [("hp", Hparams), ("weight_type", c_int32), ("token_embd", c_void_p),
                ("output_norm", c_void_p), ("layers", POINTER(LayerTensors))]


class GenStats(ctypes.Structure):
    _fields_ = [("target_calls", c_int64), ("drafted_calls", c_int64), ("proposed", c_int64),
                ("accepted", c_int64), ("target_input_tokens", c_int64), ("rewinds", c_int64),
                ("prefill_seconds", c_double), ("verify_seconds", c_double),
                ("draft_seconds", c_double), ("stop_reason", c_int32), ("next_seed", c_int32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class StreamDrafter(ctypes.Structure):
    _fields_ = [("prompt", POINTER(c_int32)), ("n_prompt", c_int32),
                ("stream", POINTER(c_int32)), ("period", c_int32)]


DRAFT_FN = ctypes.CFUNCTYPE(c_int32, c_void_p, POINTER(c_int32), c_int32, c_int32, POINTER(c_int32))
TARGET_VERIFY_FN = ctypes.CFUNCTYPE(c_int32, c_void_p, POINTER(c_int32), c_int32, POINTER(c_int32),
                                    c_int32, c_float, POINTER(c_int32), POINTER(c_int32))


class Target(ctypes.Structure):
    _fields_ = [("self", c_void_p), ("verify", TARGET_VERIFY_FN), ("past", POINTER(c_int32)),
                ("max_seq", c_int32), ("vocab", c_int32)]


COMMIT_FN = ctypes.CFUNCTYPE(None, c_void_p, POINTER(c_int32), c_int32, c_int32, c_int32)

# name -> (restype, argtypes)
SIGNATURES = {
    "mtg_abi_version": (c_int32, []),
    "mtg_create": (c_int32, [POINTER(ModelDesc), c_int32, c_int32, POINTER(c_void_p)]),
    "mtg_destroy": (None, [c_void_p]),
    "mtg_last_error": (ctypes.c_char_p, [c_void_p]),
    "mtg_past_len": (c_int32, [c_void_p]),
    "mtg_remaining": (c_int32, [c_void_p]),
    "mtg_rewind": (c_int32, [c_void_p, c_int32]),
    "mtg_embed": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "mtg_prefill": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "mtg_prefill_mode": (c_int32, [c_void_p, c_int32]),
    "mtg_last_prefill_ms": (c_double, [c_void_p]),
    "mtg_append": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "mtg_logits": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "mtg_verify": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_float, c_void_p,
                             c_void_p, c_void_p, c_void_p]),
    "mtg_kv_write": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32]),
    "mtg_kv_read": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32]),
    "mtg_generate": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_float, c_int32,
                               c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int32),
                               POINTER(GenStats)]),
    "mtg_generate_device": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                      c_float, c_int32, c_void_p, POINTER(c_int32), POINTER(GenStats)]),
    "mtg_generate_device_stream": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                             c_float, c_int32, c_void_p, c_void_p, POINTER(c_int32),
                                             POINTER(GenStats)]),
    "mtg_generate_from": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                    c_int32, c_float, c_int32, c_void_p, c_void_p, c_void_p,
                                    c_void_p, POINTER(c_int32), POINTER(GenStats)]),
    "mtg_speculative_run": (c_int32, [POINTER(Target), c_int32, c_void_p, c_int32, c_int32, c_int32,
                                      c_int32, c_float, c_int32, c_void_p, c_void_p, c_void_p,
                                      c_void_p, POINTER(c_int32), POINTER(GenStats)]),
    "mtg_stream_draft": (c_int32, [c_void_p, POINTER(c_int32), c_int32, c_int32, POINTER(c_int32)]),
    "mtg_set_exec_mode": (c_int32, [c_void_p, c_int32]),
    "mtg_exec_mode": (c_int32, [c_void_p]),
    "mtg_debug_copy": (c_int32, [c_void_p, c_int32, c_void_p, ctypes.c_size_t]),
    "mtg_debug_abort_next_step": (c_int32, [c_void_p]),
    "mtg_debug_wait_limit": (c_int32, [c_void_p, c_int32]),
    "mtg_step_fallbacks": (c_int64, [c_void_p]),
    "mtg_set_step_max_keys": (c_int32, [c_void_p, c_int32]),
    "mtg_step_kernel_runs": (c_int64, [c_void_p]),
    "mtg_step_profile": (c_int32, [c_void_p, c_int32]),
    "mtg_launch_timing": (c_int32, [c_void_p, c_int32]),
    "mtg_launch_timing_read": (c_int32, [c_void_p, POINTER(c_double), POINTER(c_int64),
                                         POINTER(c_int64), POINTER(c_int64)]),
    "mtg_step_profile_read": (c_int32, [c_void_p, c_void_p, c_int32]),
    "mtg_ngram_draft": (c_int32, [c_void_p, c_int32, c_int32, c_void_p]),
    "mtg_greedy_choice": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_float]),
    "mtg_q8_pack": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_void_p)]),
    "mtg_q8_free": (None, [c_void_p]),
    "mtg_q8_unpack": (c_int32, [c_void_p, c_void_p]),
    "mtg_q8_mul_mat_dev": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "mtg_q8_mul_mat_dev_noalloc": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
    "mtg_causal_context_dev": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                         c_int32, c_void_p]),
    "mtg_gguf_open": (c_int32, [ctypes.c_char_p, POINTER(c_void_p)]),
    "mtg_gguf_close": (None, [c_void_p]),
    "mtg_gguf_error": (ctypes.c_char_p, [c_void_p]),
    "mtg_gguf_n_tensors": (c_int64, [c_void_p]),
    "mtg_gguf_tensor": (c_int32, [c_void_p, ctypes.c_char_p, POINTER(c_int32), POINTER(c_int64),
                                  POINTER(c_void_p), POINTER(ctypes.c_size_t)]),
    "mtg_gguf_model": (POINTER(ModelDesc), [c_void_p]),
    "mtg_create_from_gguf": (c_int32, [ctypes.c_char_p, c_int32, c_int32, POINTER(c_void_p)]),
    "mtg_synth_create": (c_int32, [POINTER(Hparams), c_int32, c_uint64, c_float, c_float,
                                   POINTER(c_void_p)]),
    "mtg_synth_free": (None, [c_void_p]),
    "mtg_synth_desc": (POINTER(ModelDesc), [c_void_p]),
    "mtg_normal_fill": (None, [c_uint64, c_uint64, c_void_p, ctypes.c_size_t]),
    "mtg_quantize_q8_0_weight": (None, [c_void_p, c_int64, c_void_p]),
    "mtg_quantize_q4_k": (None, [c_void_p, c_int64, c_void_p]),
    "mtg_dequantize": (None, [c_int32, c_void_p, c_int64, c_void_p]),
    "mtg_row_bytes": (ctypes.c_size_t, [c_int32, c_int64]),
    "mtg_f32_to_f16": (c_uint16, [c_float]),
    "mtg_f16_to_f32": (c_float, [c_uint16]),
}

# ---- Whisper encoder + audio adaptor (mtg_encoder_*) ----
class EncoderHparams(ctypes.Structure):
    _fields_ = [("n_mels", c_int32), ("n_frames", c_int32), ("d_model", c_int32), ("n_layers", c_int32),
                ("n_heads", c_int32), ("ffn", c_int32), ("merge", c_int32), ("hidden", c_int32),
                ("adaptor_eps", c_float)]


class EncoderLayer(ctypes.Structure):
    _fields_ = [("attn_ln_w", c_void_p), ("attn_ln_b", c_void_p), ("q_w", c_void_p), ("k_w", c_void_p),
                ("v_w", c_void_p), ("o_w", c_void_p), ("q_b", c_void_p), ("v_b", c_void_p), ("o_b", c_void_p),
                ("ffn_ln_w", c_void_p), ("ffn_ln_b", c_void_p), ("fc1_w", c_void_p), ("fc1_b", c_void_p),
                ("fc2_w", c_void_p), ("fc2_b", c_void_p)]


class EncoderDesc(ctypes.Structure):
    _fields_ = [("hp", EncoderHparams), ("weight_type", c_int32), ("conv1_w", c_void_p), ("conv1_b", c_void_p),
                ("conv2_w", c_void_p), ("conv2_b", c_void_p), ("pos_embd", c_void_p), ("ln_post_w", c_void_p),
                ("ln_post_b", c_void_p), ("layers", POINTER(EncoderLayer)), ("ad_fc1_w", c_void_p),
                ("ad_fc1_b", c_void_p), ("ad_fc2_w", c_void_p), ("ad_fc2_b", c_void_p), ("ad_ln_w", c_void_p),
                ("ad_ln_b", c_void_p)]


ENCODER_DEFAULTS = dict(n_mels=80, n_frames=3000, d_model=1024, n_layers=24, n_heads=16, ffn=4096, merge=4,
                        hidden=1024, adaptor_eps=1e-6)

SIGNATURES.update({
    "mtg_encoder_create": (c_int32, [POINTER(EncoderDesc), POINTER(c_void_p)]),
    "mtg_encoder_destroy": (None, [c_void_p]),
    "mtg_encoder_error": (ctypes.c_char_p, [c_void_p]),
    "mtg_encoder_encode": (c_int32, [c_void_p, c_void_p, c_void_p, POINTER(c_int32)]),
    "mtg_encoder_adapt": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, POINTER(c_int32)]),
    "mtg_encoder_last_ms": (c_double, [c_void_p]),
    "mtg_gguf_encoder": (POINTER(EncoderDesc), [c_void_p]),
    "mtg_encoder_create_from_gguf": (c_int32, [ctypes.c_char_p, POINTER(c_void_p)]),
})

_lib = None


class MtgError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("mtg error %d: %s" % (code, msg))
        self.code = code


def lib():
    """Load libmtg.so (built by __graft_entry__.build()); raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError("libmtg.so is not built: run __graft_entry__.build() (%s)" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ptr(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def make_hparams(**kw):
    d = dict(QWEN3_0_6B)
    d.update(kw)
    return Hparams(**d)


class SynthModel:
    """Seeded synthetic Qwen3 model held in host memory (ggml block layout)."""

    def __init__(self, weight_type=TYPE_Q8_0, seed=0, std=0.02, gain_jitter=0.0, **hp):
        self.hp = make_hparams(**hp)
        out = c_void_p()
        rc = lib().mtg_synth_create(ctypes.byref(self.hp), weight_type, seed, std, gain_jitter,
                                    ctypes.byref(out))
        if rc:
            raise MtgError(rc, "synthetic model")
        self.handle = out
        self.desc = lib().mtg_synth_desc(out)
        self.weight_type = weight_type

    def close(self):
        if self.handle:
            lib().mtg_synth_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def matrix(self, ptr_, k, n):
        """Copy of one weight matrix's raw block bytes (n rows of k)."""
        nb = lib().mtg_row_bytes(self.weight_type, k) * n
        return np.frombuffer(ctypes.string_at(ptr_, nb), dtype=np.uint8).copy()

    def dequant_rows(self, ptr_, k, rows):
        rb = lib().mtg_row_bytes(self.weight_type, k)
        out = np.empty((len(rows), k), np.float32)
        for i, r in enumerate(rows):
            raw = ctypes.string_at(ptr_ + int(r) * rb, rb)
            lib().mtg_dequantize(self.weight_type, raw, k, ptr(out[i]))
        return out


class GgufModel:
    """A mapped GGUF file (mtg_gguf) and its decoder description (decoder=False:
    the file is not required to hold a decoder)."""

    def __init__(self, path, decoder=True):
        out = c_void_p()
        rc = lib().mtg_gguf_open(os.fsencode(path), ctypes.byref(out))
        if rc:
            raise MtgError(rc, lib().mtg_gguf_error(None).decode())
        self.handle = out
        if not decoder:
            self.desc = self.hp = self.weight_type = None
            return
        d = lib().mtg_gguf_model(out)
        if not d:
            msg = lib().mtg_gguf_error(out).decode()
            self.close()
            raise MtgError(ERR_INVALID, msg)
        self.desc = d
        self.hp = d.contents.hp
        self.weight_type = d.contents.weight_type

    def encoder(self):
        """The file's encoder + adaptor description (mtg_gguf_encoder)."""
        d = lib().mtg_gguf_encoder(self.handle)
        if not d:
            raise MtgError(ERR_INVALID, lib().mtg_gguf_error(self.handle).decode())
        return d

    def tensor(self, name):
        """(ggml type, ne[4], raw bytes) of one tensor."""
        t, ne, data, nb = c_int32(), (c_int64 * 4)(), c_void_p(), ctypes.c_size_t()
        rc = lib().mtg_gguf_tensor(self.handle, name.encode(), ctypes.byref(t), ne, ctypes.byref(data),
                                   ctypes.byref(nb))
        if rc:
            raise KeyError(name)
        return t.value, list(ne), ctypes.string_at(data, nb.value)

    def close(self):
        if self.handle:
            lib().mtg_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """Device decoder context (mtg_ctx)."""

    def __init__(self, model, max_seq, kv_type=TYPE_F32):
        self.hp = model.hp
        out = c_void_p()
        rc = lib().mtg_create(model.desc, max_seq, kv_type, ctypes.byref(out))
        if rc:
            raise MtgError(rc, lib().mtg_last_error(None).decode())
        self.ctx = out
        self.kv_type = kv_type
        self.max_seq = max_seq

    @classmethod
    def from_gguf(cls, path, max_seq, kv_type=TYPE_F32):
        """A decoder whose weights come from a GGUF file (mtg_create_from_gguf);
        the file's hyper-parameters are read with mtg_gguf_open first."""
        g = GgufModel(path)
        hp = Hparams()
        ctypes.memmove(ctypes.byref(hp), ctypes.byref(g.hp), ctypes.sizeof(Hparams))
        g.close()
        self = cls.__new__(cls)
        self.hp = hp
        out = c_void_p()
        rc = lib().mtg_create_from_gguf(os.fsencode(path), max_seq, kv_type, ctypes.byref(out))
        if rc:
            raise MtgError(rc, lib().mtg_last_error(None).decode())
        self.ctx = out
        self.kv_type = kv_type
        self.max_seq = max_seq
        return self

    def _chk(self, rc):
        if rc:
            raise MtgError(rc, lib().mtg_last_error(self.ctx).decode())

    def close(self):
        if self.ctx:
            lib().mtg_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def past_len(self):
        return lib().mtg_past_len(self.ctx)

    def rewind(self, pos):
        self._chk(lib().mtg_rewind(self.ctx, pos))

    def set_exec(self, mode):
        self._chk(lib().mtg_set_exec_mode(self.ctx, mode))

    def debug_abort_next_step(self):
        self._chk(lib().mtg_debug_abort_next_step(self.ctx))

    def debug_wait_limit(self, polls):
        self._chk(lib().mtg_debug_wait_limit(self.ctx, polls))

    @property
    def step_fallbacks(self):
        return lib().mtg_step_fallbacks(self.ctx)

    def set_step_max_keys(self, max_keys):
        """KV length beyond which steps take the per-op graph (<= 0: the default)."""
        self._chk(lib().mtg_set_step_max_keys(self.ctx, max_keys))

    @property
    def step_kernel_runs(self):
        return lib().mtg_step_kernel_runs(self.ctx)

    def debug_buffer(self, which, width):
        out = np.empty((MAX_BATCH, width), np.float32)
        self._chk(lib().mtg_debug_copy(self.ctx, which, ptr(out), out.nbytes))
        return out

    def step_profile(self, on):
        self._chk(lib().mtg_step_profile(self.ctx, 1 if on else 0))

    def launch_timing(self, on):
        self._chk(lib().mtg_launch_timing(self.ctx, 1 if on else 0))

    def launch_timing_read(self):
        """(total ms, launches, sum of past_len, sum of rows) of the timed steps."""
        ms, n, ps, rs = c_double(), c_int64(), c_int64(), c_int64()
        self._chk(lib().mtg_launch_timing_read(self.ctx, ctypes.byref(ms), ctypes.byref(n),
                                               ctypes.byref(ps), ctypes.byref(rs)))
        return ms.value, n.value, ps.value, rs.value

    def step_marks(self):
        out = np.zeros(PROFILE_SLOTS, np.uint64)
        n = lib().mtg_step_profile_read(self.ctx, ptr(out), PROFILE_SLOTS)
        return out[:n].astype(np.int64)

    @property
    def exec_mode(self):
        return lib().mtg_exec_mode(self.ctx)

    def embed(self, ids):
        ids = i32(ids)
        out = np.empty((len(ids), self.hp.hidden), np.float32)
        self._chk(lib().mtg_embed(self.ctx, ptr(ids), len(ids), ptr(out)))
        return out

    def prefill(self, embeds, want_hidden=True):
        embeds = f32(embeds)
        S = embeds.shape[0]
        hid = np.empty((S, self.hp.hidden), np.float32) if want_hidden else None
        self._chk(lib().mtg_prefill(self.ctx, ptr(embeds), S, ptr(hid)))
        return hid

    def prefill_mode(self, blocks):
        self._chk(lib().mtg_prefill_mode(self.ctx, 1 if blocks else 0))

    @property
    def last_prefill_ms(self):
        return lib().mtg_last_prefill_ms(self.ctx)

    def append(self, embeds):
        embeds = f32(embeds)
        T = embeds.shape[0]
        hid = np.empty((T, self.hp.hidden), np.float32)
        self._chk(lib().mtg_append(self.ctx, ptr(embeds), T, ptr(hid)))
        return hid

    def logits(self, hidden):
        hidden = f32(hidden)
        T = hidden.shape[0]
        out = np.empty((T, self.hp.vocab), np.float32)
        self._chk(lib().mtg_logits(self.ctx, ptr(hidden), T, ptr(out)))
        return out

    def verify(self, tokens, history=(), penalty=1.0, want_hidden=False, want_logits=False):
        tokens = i32(tokens)
        T = len(tokens)
        hist = i32(history)
        choice = np.empty(T, np.int32)
        n_match = np.zeros(1, np.int32)
        hid = np.empty((T, self.hp.hidden), np.float32) if want_hidden else None
        lg = np.empty((T, self.hp.vocab), np.float32) if want_logits else None
        self._chk(lib().mtg_verify(self.ctx, ptr(tokens), T, ptr(hist) if len(hist) else None,
                                   len(hist), penalty, ptr(choice), ptr(n_match), ptr(hid), ptr(lg)))
        return choice, int(n_match[0]), hid, lg

    def kv_dtype(self):
        return np.float32 if self.kv_type == TYPE_F32 else np.float16

    def kv_read(self, n_pos):
        shape = (self.hp.n_layers, self.hp.n_kv_heads, n_pos, self.hp.head_dim)
        k = np.empty(shape, self.kv_dtype())
        v = np.empty(shape, self.kv_dtype())
        self._chk(lib().mtg_kv_read(self.ctx, ptr(k), ptr(v), n_pos))
        return k, v

    def kv_write(self, k, v):
        k = np.ascontiguousarray(k, self.kv_dtype())
        v = np.ascontiguousarray(v, self.kv_dtype())
        self._chk(lib().mtg_kv_write(self.ctx, ptr(k), ptr(v), k.shape[2]))

    def generate_from(self, first_seed, max_new, max_steps=0, eos=-1, penalty=1.0, max_draft=4,
                      draft=None, user=None, prior=()):
        """Run the speculative controller; draft is None (reference n-gram), a
        (c function pointer, user pointer) pair, or a Python callable."""
        out = np.empty(max_new, np.int32)
        n = c_int32(0)
        st = GenStats()
        prior = i32(prior)
        keep = None
        fn = None
        if callable(draft):
            def _cb(_user, ids, n_ids, budget, dst, _f=draft):
                props = list(_f([ids[i] for i in range(n_ids)], budget))[:budget]
                for i, t in enumerate(props):
                    dst[i] = int(t)
                return len(props)
            keep = DRAFT_FN(_cb)
            fn = ctypes.cast(keep, c_void_p)
        elif draft is not None:
            fn = draft
        self._chk(lib().mtg_generate_from(self.ctx, first_seed, ptr(prior) if len(prior) else None,
                                          len(prior), max_new, max_steps, eos, penalty, max_draft,
                                          fn, None, user, ptr(out), ctypes.byref(n),
                                          ctypes.byref(st)))
        del keep
        return out[: n.value].copy(), st

    def generate_device(self, first_seed, max_new, max_steps=0, eos=-1, penalty=1.0, max_draft=4, prior=(),
                        stream=None):
        """The speculative controller on the device: the reference n-gram drafter,
        or (stream = a stream_drafter() triple) the stream drafter run by the
        controller kernel (mtg_generate_device_stream)."""
        out = np.empty(max_new, np.int32)
        n = c_int32(0)
        st = GenStats()
        prior = i32(prior)
        if stream is None:
            self._chk(lib().mtg_generate_device(self.ctx, first_seed, ptr(prior) if len(prior) else None,
                                                len(prior), max_new, max_steps, eos, penalty, max_draft, ptr(out),
                                                ctypes.byref(n), ctypes.byref(st)))
        else:
            _fn, user, _keep = stream
            self._chk(lib().mtg_generate_device_stream(self.ctx, first_seed, ptr(prior) if len(prior) else None,
                                                       len(prior), max_new, max_steps, eos, penalty, max_draft,
                                                       user, ptr(out), ctypes.byref(n), ctypes.byref(st)))
        return out[: n.value].copy(), st


def _draft_pointer(draft):
    """(function pointer, keepalive) for a Python drafter callable."""
    if draft is None:
        return None, None
    if not callable(draft):
        return draft, None

    def _cb(_user, ids, n_ids, budget, dst, _f=draft):
        props = list(_f([ids[i] for i in range(n_ids)], budget))[:budget]
        for i, t in enumerate(props):
            dst[i] = int(t)
        return len(props)
    keep = DRAFT_FN(_cb)
    return ctypes.cast(keep, c_void_p), keep


def speculative_run(verify_cb, first_seed, max_new, eos=-1, penalty=1.0, max_draft=4, past=0,
                    max_seq=1 << 20, vocab=1 << 20, draft=None, prior=(), max_steps=0,
                    commits=None):
    """Drive the library's controller (mtg_speculative_run) with a Python target:
    verify_cb(tokens, history, penalty, past) -> (choices, n_match). Returns
    (ids, stats, past)."""
    past_box = c_int32(past)

    def _verify(_self, tokens, T, hist, nh, pen, choice_out, n_match_out):
        try:
            ch, nm = verify_cb([tokens[i] for i in range(T)], [hist[i] for i in range(nh)], pen,
                               past_box.value)
        except Exception:
            return ERR_INVALID
        for i in range(T):
            choice_out[i] = int(ch[i])
        n_match_out[0] = int(nm)
        return OK
    vfn = TARGET_VERIFY_FN(_verify)
    tg = Target(None, vfn, ctypes.pointer(past_box), max_seq, vocab)
    fn, keep = _draft_pointer(draft)
    cfn = None
    if commits is not None:
        def _commit(_u, ids, n, past_len, stopped):
            commits.append(([ids[i] for i in range(n)], past_len, stopped))
        cfn_keep = COMMIT_FN(_commit)
        cfn = ctypes.cast(cfn_keep, c_void_p)
    out = np.empty(max_new, np.int32)
    n = c_int32(0)
    st = GenStats()
    prior = i32(prior)
    rc = lib().mtg_speculative_run(ctypes.byref(tg), first_seed, ptr(prior) if len(prior) else None,
                                   len(prior), max_new, max_steps, eos, penalty, max_draft, fn, cfn,
                                   None, ptr(out), ctypes.byref(n), ctypes.byref(st))
    del keep, vfn
    if rc:
        raise MtgError(rc, "speculative_run")
    return [int(x) for x in out[: n.value]], st, past_box.value


def stream_drafter(prompt, stream):
    """(function pointer, user pointer, keepalive) for mtg_stream_draft."""
    prompt = i32(prompt)
    stream = i32(stream)
    d = StreamDrafter(prompt.ctypes.data_as(POINTER(c_int32)), len(prompt),
                      stream.ctypes.data_as(POINTER(c_int32)), len(stream))
    fn = ctypes.cast(lib().mtg_stream_draft, c_void_p)
    return fn, ctypes.cast(ctypes.pointer(d), c_void_p), (prompt, stream, d)


def ngram_draft(history, maximum):
    h = i32(history)
    out = np.zeros(max(maximum, 1), np.int32)
    n = lib().mtg_ngram_draft(ptr(h) if len(h) else None, len(h), maximum, ptr(out))
    return [int(x) for x in out[:n]]


def greedy_choice(raw, history, penalty):
    raw = f32(raw)
    h = i32(history)
    return int(lib().mtg_greedy_choice(ptr(raw), len(raw), ptr(h) if len(h) else None, len(h),
                                       penalty))


def normal(seed, first, n):
    out = np.empty(n, np.float32)
    lib().mtg_normal_fill(seed, first, ptr(out), n)
    return out


class SynthEncoder:
    """Seeded synthetic Whisper encoder + adaptor in host memory: f32 conv stem,
    positional embedding, norms and biases; q8_0 (the converter's q8_0 dtype), f16
    (its f16 dtype) or q4_K (`cli quantize q4_k`) projection / FFN / adaptor
    matrices, from the shared normal stream."""

    def __init__(self, seed=0, std=0.02, wtype=TYPE_Q8_0, **hp):
        d = dict(ENCODER_DEFAULTS)
        d.update(hp)
        self.hp = EncoderHparams(**d)
        self._keep = []
        self._next = 0
        self.seed = seed
        self.wtype = wtype
        h = self.hp
        D, F, M, H, IN = h.d_model, h.ffn, h.n_mels, h.hidden, h.d_model * h.merge
        R = (h.n_frames - 1) // 2 + 1
        self.rows = R
        desc = EncoderDesc()
        desc.hp = self.hp
        desc.weight_type = wtype
        desc.conv1_w = self._f(D * M * 3, std)
        desc.conv1_b = self._f(D, std)
        desc.conv2_w = self._f(D * D * 3, std)
        desc.conv2_b = self._f(D, std)
        desc.pos_embd = self._f(R * D, 0.2)
        desc.ln_post_w = self._f(D, 0.05, 1.0)
        desc.ln_post_b = self._f(D, 0.05)
        layers = (EncoderLayer * max(1, h.n_layers))()
        for i in range(h.n_layers):
            L = layers[i]
            L.attn_ln_w, L.attn_ln_b = self._f(D, 0.05, 1.0), self._f(D, 0.05)
            L.q_w, L.k_w, L.v_w, L.o_w = (self._q(D, D, std) for _ in range(4))
            L.q_b, L.v_b, L.o_b = (self._f(D, std) for _ in range(3))
            L.ffn_ln_w, L.ffn_ln_b = self._f(D, 0.05, 1.0), self._f(D, 0.05)
            L.fc1_w, L.fc1_b = self._q(F, D, std), self._f(F, std)
            L.fc2_w, L.fc2_b = self._q(D, F, std), self._f(D, std)
        self._keep.append(layers)
        desc.layers = layers
        desc.ad_fc1_w, desc.ad_fc1_b = self._q(H, IN, std), self._f(H, std)
        desc.ad_fc2_w, desc.ad_fc2_b = self._q(H, H, std), self._f(H, std)
        desc.ad_ln_w, desc.ad_ln_b = self._f(H, 0.05, 1.0), self._f(H, 0.05)
        self.desc = desc

    def _normal(self, n):
        out = normal(self.seed, self._next, n)
        self._next += n
        return out

    def _f(self, n, std, mean=0.0):
        a = (self._normal(n) * np.float32(std) + np.float32(mean)).astype(np.float32)
        self._keep.append(a)
        return a.ctypes.data

    def _q(self, n, k, std):
        x = (self._normal(n * k) * np.float32(std)).astype(np.float32)
        if self.wtype == TYPE_F16:
            blocks = x.astype(np.float16).view(np.uint8)
        elif self.wtype == TYPE_F32:
            blocks = x.view(np.uint8)
        elif self.wtype == TYPE_Q4_K:
            blocks = np.empty(n * (k // 256) * 144, np.uint8)
            lib().mtg_quantize_q4_k(ptr(x), n * k, ptr(blocks))
        else:
            blocks = np.empty(n * (k // 32) * 34, np.uint8)
            lib().mtg_quantize_q8_0_weight(ptr(x), n * k, ptr(blocks))
        blocks = np.ascontiguousarray(blocks)
        self._keep.append(blocks)
        return blocks.ctypes.data

    def mel(self, seed=1):
        """A mel chunk [n_mels][n_frames] shaped like log-mel features."""
        h = self.hp
        return (normal(seed, 0, h.n_mels * h.n_frames) * np.float32(0.5)).reshape(h.n_mels, h.n_frames)


class Encoder:
    """Device encoder + adaptor (mtg_encoder)."""

    def __init__(self, synth):
        self.hp = synth.hp
        self.rows = synth.rows
        out = c_void_p()
        rc = lib().mtg_encoder_create(ctypes.byref(synth.desc), ctypes.byref(out))
        if rc:
            raise MtgError(rc, "encoder create")
        self.h = out

    @classmethod
    def from_gguf(cls, path):
        g = GgufModel(path, decoder=False)
        hp = EncoderHparams()
        ctypes.memmove(ctypes.byref(hp), ctypes.byref(g.encoder().contents.hp), ctypes.sizeof(EncoderHparams))
        g.close()
        self = cls.__new__(cls)
        self.hp = hp
        self.rows = (hp.n_frames - 1) // 2 + 1
        out = c_void_p()
        rc = lib().mtg_encoder_create_from_gguf(os.fsencode(path), ctypes.byref(out))
        if rc:
            raise MtgError(rc, lib().mtg_gguf_error(None).decode())
        self.h = out
        return self

    def _chk(self, rc):
        if rc:
            raise MtgError(rc, lib().mtg_encoder_error(self.h).decode())

    def encode(self, mel, want_rows=True):
        mel = f32(mel)
        out = np.empty((self.rows, self.hp.d_model), np.float32) if want_rows else None
        n = c_int32(0)
        self._chk(lib().mtg_encoder_encode(self.h, ptr(mel), ptr(out), ctypes.byref(n)))
        return out

    def adapt(self, T, rows=None):
        n_out = T // self.hp.merge
        out = np.empty((max(1, n_out), self.hp.hidden), np.float32)
        n = c_int32(0)
        r = None if rows is None else f32(rows)
        self._chk(lib().mtg_encoder_adapt(self.h, ptr(r), T, ptr(out), ctypes.byref(n)))
        return out[: n.value]

    @property
    def last_ms(self):
        return lib().mtg_encoder_last_ms(self.h)

    def close(self):
        if self.h:
            lib().mtg_encoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
