"""A small GGUF (v3) writer for the loader tests: header, typed metadata,
tensor table, aligned data section, written from the published file layout
(magic "GGUF", version, tensor count, metadata count, key/value pairs, tensor
infos {name, n_dims, ne, ggml type, offset}, padding to general.alignment).
It writes a model the way the reference's converter names and types it
(scripts/convert_moss_transcribe_to_gguf.py:46-76, 242-259): decoder matrices and
token_embd.weight in the weight type, norm gains f32."""
import ctypes
import struct

import numpy as np

import mtg

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}[t]
    return struct.pack(fmt, v)


def write(path, kv, tensors, alignment=32, version=3):
    """kv: [(key, type, value)]; tensors: [(name, ggml_type, ne list, bytes)]."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for name, t, ne, data in tensors:
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, t, ne, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne)
        head += struct.pack("<IQ", t, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, t, ne, data), o in zip(tensors, offsets):
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))


def model_tensors(model, f16_norms=False):
    """The decoder tensors of a SynthModel with their GGUF names, ne and bytes."""
    hp, d = model.hp, model.desc.contents
    H, D = hp.hidden, hp.head_dim
    QN, KN, F = hp.n_heads * D, hp.n_kv_heads * D, hp.intermediate
    wt = model.weight_type

    def mat(p, k, n):
        return (wt, [k, n], ctypes.string_at(p, mtg.lib().mtg_row_bytes(wt, k) * n))

    def gain(p, n):
        v = np.frombuffer(ctypes.string_at(p, 4 * n), np.float32)
        if f16_norms:
            return (1, [n], v.astype(np.float16).tobytes())
        return (0, [n], v.tobytes())

    out = [("token_embd.weight",) + mat(d.token_embd, H, hp.vocab)]
    for i in range(hp.n_layers):
        L = d.layers[i]
        b = "qwen3.blk.%d." % i
        out += [(b + "attn_norm.weight",) + gain(L.attn_norm, H),
                (b + "attn_q.weight",) + mat(L.attn_q, H, QN),
                (b + "attn_k.weight",) + mat(L.attn_k, H, KN),
                (b + "attn_v.weight",) + mat(L.attn_v, H, KN),
                (b + "attn_o.weight",) + mat(L.attn_o, QN, H),
                (b + "attn_q_norm.weight",) + gain(L.attn_q_norm, D),
                (b + "attn_k_norm.weight",) + gain(L.attn_k_norm, D),
                (b + "ffn_norm.weight",) + gain(L.ffn_norm, H),
                (b + "ffn_gate.weight",) + mat(L.ffn_gate, H, F),
                (b + "ffn_up.weight",) + mat(L.ffn_up, H, F),
                (b + "ffn_down.weight",) + mat(L.ffn_down, F, H)]
    out.append(("qwen3.output_norm.weight",) + gain(d.output_norm, H))
    return out


def model_metadata(model, extra=()):
    hp = model.hp
    kv = [("general.architecture", STR, "moss-transcribe"),
          ("mtd.text.vocab_size", U32, hp.vocab), ("mtd.text.hidden", U32, hp.hidden),
          ("mtd.text.ffn", U32, hp.intermediate), ("mtd.text.n_layers", U32, hp.n_layers),
          ("mtd.text.n_heads", U32, hp.n_heads), ("mtd.text.n_kv_heads", U32, hp.n_kv_heads),
          ("mtd.text.head_dim", U32, hp.head_dim), ("mtd.text.rms_eps", F32, hp.rms_eps),
          ("mtd.text.rope_theta", F32, hp.rope_base),
          # keys the decoder does not read, of every kind the parser must skip
          ("tokenizer.ggml.tokens", ARR, (STR, ["<s>", "a", "bc"])),
          ("mtd.digit_token_ids", ARR, (I32, [15, 16, 17])),
          ("mtd.feat.dither", F32, 0.0), ("mtd.enable_time_marker", BOOL, True),
          ("mtd.text.max_pos", U64, 40960)]
    return kv + list(extra)


def write_model(path, model, f16_norms=False, alignment=32, extra_kv=(), edit=None):
    """Write a SynthModel as a GGUF file; edit(tensors) may alter the tensor list."""
    tensors = [(n, t, ne, data) for n, t, ne, data in model_tensors(model, f16_norms)]
    if edit is not None:
        tensors = edit(tensors)
    kv = model_metadata(model, extra_kv)
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    write(path, kv, tensors, alignment)


def encoder_tensors(syn):
    """The encoder + adaptor tensors of a SynthEncoder with their GGUF names
    (src/whisper_encoder.cpp:71-94, src/audio_adaptor.cpp:28-33)."""
    h, d = syn.hp, syn.desc
    D, F, M, H, IN = h.d_model, h.ffn, h.n_mels, h.hidden, h.d_model * h.merge
    R = syn.rows
    wt = getattr(syn, "wtype", mtg.TYPE_Q8_0)  # the matrices' type (q8_0, f16, f32 or q4_K)
    rb = lambda k: mtg.lib().mtg_row_bytes(wt, k)

    def f32(p, ne):
        return (0, ne, ctypes.string_at(p, 4 * int(np.prod(ne))))

    def q8(p, k, n):
        return (wt, [k, n], ctypes.string_at(p, rb(k) * n))

    out = [("enc.conv1.w",) + f32(d.conv1_w, [3, M, D]), ("enc.conv1.b",) + f32(d.conv1_b, [D]),
           ("enc.conv2.w",) + f32(d.conv2_w, [3, D, D]), ("enc.conv2.b",) + f32(d.conv2_b, [D]),
           ("enc.pos_embd",) + f32(d.pos_embd, [D, R])]
    for i in range(h.n_layers):
        L = d.layers[i]
        b = "enc.blk.%d." % i
        out += [(b + "attn_ln.w",) + f32(L.attn_ln_w, [D]), (b + "attn_ln.b",) + f32(L.attn_ln_b, [D]),
                (b + "attn_q.w",) + q8(L.q_w, D, D), (b + "attn_q.b",) + f32(L.q_b, [D]),
                (b + "attn_k.w",) + q8(L.k_w, D, D), (b + "attn_v.w",) + q8(L.v_w, D, D),
                (b + "attn_v.b",) + f32(L.v_b, [D]), (b + "attn_out.w",) + q8(L.o_w, D, D),
                (b + "attn_out.b",) + f32(L.o_b, [D]), (b + "ffn_ln.w",) + f32(L.ffn_ln_w, [D]),
                (b + "ffn_ln.b",) + f32(L.ffn_ln_b, [D]), (b + "ffn_1.w",) + q8(L.fc1_w, D, F),
                (b + "ffn_1.b",) + f32(L.fc1_b, [F]), (b + "ffn_2.w",) + q8(L.fc2_w, F, D),
                (b + "ffn_2.b",) + f32(L.fc2_b, [D])]
    out += [("enc.ln_post.w",) + f32(d.ln_post_w, [D]), ("enc.ln_post.b",) + f32(d.ln_post_b, [D]),
            ("adaptor.fc1.w",) + q8(d.ad_fc1_w, IN, H), ("adaptor.fc1.b",) + f32(d.ad_fc1_b, [H]),
            ("adaptor.fc2.w",) + q8(d.ad_fc2_w, H, H), ("adaptor.fc2.b",) + f32(d.ad_fc2_b, [H]),
            ("adaptor.ln.w",) + f32(d.ad_ln_w, [H]), ("adaptor.ln.b",) + f32(d.ad_ln_b, [H])]
    return out


def encoder_metadata(syn):
    h = syn.hp
    return [("mtd.audio.mel_bins", U32, h.n_mels), ("mtd.audio.d_model", U32, h.d_model),
            ("mtd.audio.n_layers", U32, h.n_layers), ("mtd.audio.n_heads", U32, h.n_heads),
            ("mtd.audio.ffn", U32, h.ffn), ("mtd.audio.max_src_pos", U32, syn.rows),
            ("mtd.audio_merge_size", U32, h.merge), ("mtd.adaptor_input_dim", U32, h.d_model * h.merge),
            ("mtd.adaptor_norm_eps", F32, h.adaptor_eps), ("mtd.audio.act", STR, "gelu")]


def write_encoder(path, syn, model=None, edit=None):
    """A GGUF file with a SynthEncoder's tensors (and a SynthModel's decoder, if given)."""
    tensors = encoder_tensors(syn)
    kv = encoder_metadata(syn) + [("mtd.text.hidden", U32, syn.hp.hidden)]
    if model is not None:
        tensors = model_tensors(model) + tensors
        kv = model_metadata(model) + encoder_metadata(syn)
    if edit is not None:
        tensors = edit(tensors)
    write(path, kv, tensors)
