"""The GGUF loader (csrc/gguf.cpp; reference ModelLoader::load / read_config,
src/model_loader.cpp:21-169) on the CPU: files written by tests/gguf_writer.py
from a seeded synthetic model must give back every tensor byte for byte, the
hyper-parameters, the weight type and f32 norm gains (f16 ones widened); damaged
or foreign files must fail with a reason, never crash. The device decoder built
from a file is checked against the one built from the model in
test_gpu_gguf.py."""
import ctypes
import os
import struct

import numpy as np
import pytest

import gguf_writer
import mtg


@pytest.fixture(scope="module", params=[mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K], ids=["q8_0", "f16", "f32", "q4_K"])
def model(request):
    m = mtg.SynthModel(request.param, seed=7, std=0.02, gain_jitter=0.05, n_layers=2, vocab=2048)
    yield m
    m.close()


def _desc_bytes(desc, hp, wt):
    """Every tensor of a model description as bytes, in a fixed order."""
    d = desc.contents
    H, D = hp.hidden, hp.head_dim
    QN, KN, F = hp.n_heads * D, hp.n_kv_heads * D, hp.intermediate
    rb = lambda k: mtg.lib().mtg_row_bytes(wt, k)
    out = [ctypes.string_at(d.token_embd, rb(H) * hp.vocab), ctypes.string_at(d.output_norm, 4 * H)]
    for i in range(hp.n_layers):
        L = d.layers[i]
        out += [ctypes.string_at(L.attn_norm, 4 * H), ctypes.string_at(L.attn_q, rb(H) * QN),
                ctypes.string_at(L.attn_k, rb(H) * KN), ctypes.string_at(L.attn_v, rb(H) * KN),
                ctypes.string_at(L.attn_o, rb(QN) * H), ctypes.string_at(L.attn_q_norm, 4 * D),
                ctypes.string_at(L.attn_k_norm, 4 * D), ctypes.string_at(L.ffn_norm, 4 * H),
                ctypes.string_at(L.ffn_gate, rb(H) * F), ctypes.string_at(L.ffn_up, rb(H) * F),
                ctypes.string_at(L.ffn_down, rb(F) * H)]
    return out


@pytest.mark.parametrize("alignment", [32, 64])
def test_round_trip(model, tmp_path, alignment):
    path = str(tmp_path / "m.gguf")
    gguf_writer.write_model(path, model, alignment=alignment)
    g = mtg.GgufModel(path)
    hp = g.hp
    for f in ("hidden", "n_heads", "n_kv_heads", "head_dim", "intermediate", "n_layers", "vocab"):
        assert getattr(hp, f) == getattr(model.hp, f), f
    assert hp.rms_eps == np.float32(model.hp.rms_eps) and hp.rope_base == np.float32(model.hp.rope_base)
    assert g.weight_type == model.weight_type
    assert mtg.lib().mtg_gguf_n_tensors(g.handle) == 2 + 11 * model.hp.n_layers
    got = _desc_bytes(g.desc, hp, g.weight_type)
    want = _desc_bytes(model.desc, model.hp, model.weight_type)
    assert len(got) == len(want)
    for i, (a, b) in enumerate(zip(got, want)):
        assert a == b, i
    t, ne, raw = g.tensor("qwen3.blk.1.ffn_down.weight")
    assert t == model.weight_type and ne[:2] == [model.hp.intermediate, model.hp.hidden]
    g.close()


def test_f16_norm_gains_are_widened(model, tmp_path):
    path = str(tmp_path / "m16.gguf")
    gguf_writer.write_model(path, model, f16_norms=True)
    g = mtg.GgufModel(path)
    H = model.hp.hidden
    got = np.frombuffer(ctypes.string_at(g.desc.contents.layers[0].attn_norm, 4 * H), np.float32)
    src = np.frombuffer(ctypes.string_at(model.desc.contents.layers[0].attn_norm, 4 * H), np.float32)
    assert np.array_equal(got, src.astype(np.float16).astype(np.float32))
    g.close()


def test_defaults_when_metadata_is_absent(tmp_path):
    """read_config's defaults (src/model_loader.cpp:118-128) are the Qwen3-0.6B
    dims: a file without mtd.text.* keys is read with them, so a 2-layer file
    fails on the missing layer 2 tensors, with the name in the message."""
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=8, n_layers=2, vocab=151936)
    path = str(tmp_path / "nometa.gguf")
    gguf_writer.write(path, [], [(n, t, ne, d) for n, t, ne, d in gguf_writer.model_tensors(m)])
    with pytest.raises(mtg.MtgError) as e:
        mtg.GgufModel(path)
    assert "qwen3.blk.2." in str(e.value)
    m.close()


def _expect_failure(path, needle):
    with pytest.raises(mtg.MtgError) as e:
        mtg.GgufModel(path)
    assert needle in str(e.value), str(e.value)
    out = ctypes.c_void_p()
    rc = mtg.lib().mtg_create_from_gguf(os.fsencode(path), 64, mtg.TYPE_F32, ctypes.byref(out))
    assert rc != 0 and not out.value
    assert needle in mtg.lib().mtg_last_error(None).decode()


def test_damaged_and_foreign_files_fail_with_a_reason(tmp_path):
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=9, n_layers=1, vocab=512)
    good = str(tmp_path / "good.gguf")
    gguf_writer.write_model(good, m)
    raw = open(good, "rb").read()
    # bad magic
    p = str(tmp_path / "magic.gguf")
    open(p, "wb").write(b"GGUX" + raw[4:])
    _expect_failure(p, "bad magic")
    # truncated inside the metadata, and inside the tensor data
    for cut, needle in ((200, "truncated"), (len(raw) - 1000, "outside the file")):
        p = str(tmp_path / ("cut%d.gguf" % cut))
        open(p, "wb").write(raw[:cut])
        _expect_failure(p, needle)
    # a missing tensor
    p = str(tmp_path / "missing.gguf")
    gguf_writer.write_model(p, m, edit=lambda ts: [t for t in ts if t[0] != "qwen3.blk.0.attn_o.weight"])
    _expect_failure(p, "missing tensor qwen3.blk.0.attn_o.weight")
    # a wrong shape
    def transpose_q(ts):
        return [(n, t, ne[::-1] if n == "qwen3.blk.0.attn_q.weight" else ne, d) for n, t, ne, d in ts]
    p = str(tmp_path / "shape.gguf")
    gguf_writer.write_model(p, m, edit=transpose_q)
    _expect_failure(p, "shape")
    # a matrix of another type than token_embd (f16 bytes of the same size class)
    def f16_gate(ts):
        out = []
        for n, t, ne, d in ts:
            if n == "qwen3.blk.0.ffn_gate.weight":
                t, d = 1, np.zeros(ne[0] * ne[1], np.float16).tobytes()
            out.append((n, t, ne, d))
        return out
    p = str(tmp_path / "mixed.gguf")
    gguf_writer.write_model(p, m, edit=f16_gate)
    _expect_failure(p, "mixed weight types")
    # an unsupported weight type everywhere (Q6_K geometry: 210 bytes per 256)
    def q6k(ts):
        out = []
        for n, t, ne, d in ts:
            if t == 8:
                t, d = 14, b"\0" * (ne[0] // 256 * 210 * ne[1])
            out.append((n, t, ne, d))
        return out
    p = str(tmp_path / "q6k.gguf")
    gguf_writer.write_model(p, m, edit=q6k)
    _expect_failure(p, "not supported")
    # a data offset that is not aligned
    p = str(tmp_path / "align.gguf")
    gguf_writer.write_model(p, m)
    b = bytearray(open(p, "rb").read())
    name = b"qwen3.output_norm.weight"
    i = b.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    n_dims = struct.unpack_from("<I", b, i)[0]
    off_pos = i + 4 + 8 * n_dims + 4
    struct.pack_into("<Q", b, off_pos, struct.unpack_from("<Q", b, off_pos)[0] + 4)
    open(p, "wb").write(bytes(b))
    _expect_failure(p, "outside the file")
    # not a file
    with pytest.raises(mtg.MtgError):
        mtg.GgufModel(str(tmp_path / "absent.gguf"))
    m.close()


def _enc_bytes(desc, syn):
    h = syn.hp
    D, F, M, H, IN = h.d_model, h.ffn, h.n_mels, h.hidden, h.d_model * h.merge
    rb = lambda k: mtg.lib().mtg_row_bytes(syn.wtype, k)
    d = desc.contents if hasattr(desc, "contents") else desc
    fs = lambda p, n: ctypes.string_at(p, 4 * n)
    out = [fs(d.conv1_w, D * M * 3), fs(d.conv1_b, D), fs(d.conv2_w, D * D * 3), fs(d.conv2_b, D),
           fs(d.pos_embd, syn.rows * D), fs(d.ln_post_w, D), fs(d.ln_post_b, D),
           ctypes.string_at(d.ad_fc1_w, rb(IN) * H), fs(d.ad_fc1_b, H), ctypes.string_at(d.ad_fc2_w, rb(H) * H),
           fs(d.ad_fc2_b, H), fs(d.ad_ln_w, H), fs(d.ad_ln_b, H)]
    for i in range(h.n_layers):
        L = d.layers[i]
        out += [fs(L.attn_ln_w, D), fs(L.attn_ln_b, D), ctypes.string_at(L.q_w, rb(D) * D),
                ctypes.string_at(L.k_w, rb(D) * D), ctypes.string_at(L.v_w, rb(D) * D),
                ctypes.string_at(L.o_w, rb(D) * D), fs(L.q_b, D), fs(L.v_b, D), fs(L.o_b, D), fs(L.ffn_ln_w, D),
                fs(L.ffn_ln_b, D), ctypes.string_at(L.fc1_w, rb(D) * F), fs(L.fc1_b, F),
                ctypes.string_at(L.fc2_w, rb(F) * D), fs(L.fc2_b, D)]
    return out


def test_encoder_tensors_round_trip(tmp_path):
    """The encoder + adaptor of a file with the decoder too (the converter's
    layout): every tensor byte for byte, the mtd.audio.* hyper-parameters, and
    the reference defaults when the keys are absent."""
    syn = mtg.SynthEncoder(seed=4, n_mels=16, n_frames=96, d_model=128, n_layers=2, n_heads=2, ffn=256, merge=4,
                           hidden=128)
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=2, n_layers=1, vocab=512, hidden=128, n_heads=2, n_kv_heads=1,
                       intermediate=256)
    path = str(tmp_path / "full.gguf")
    gguf_writer.write_encoder(path, syn, model=m)
    g = mtg.GgufModel(path)
    e = g.encoder().contents
    for f in ("n_mels", "n_frames", "d_model", "n_layers", "n_heads", "ffn", "merge", "hidden"):
        assert getattr(e.hp, f) == getattr(syn.hp, f), f
    assert e.hp.adaptor_eps == np.float32(syn.hp.adaptor_eps) and e.weight_type == mtg.TYPE_Q8_0
    got, want = _enc_bytes(e, syn), _enc_bytes(syn.desc, syn)
    assert len(got) == len(want)
    for i, (a, b) in enumerate(zip(got, want)):
        assert a == b, i
    g.close()
    # without the mtd.audio.* keys: read_config's defaults (24 layers of d 1024)
    p2 = str(tmp_path / "nokeys.gguf")
    gguf_writer.write(p2, [], gguf_writer.encoder_tensors(syn))
    out = ctypes.c_void_p()
    assert mtg.lib().mtg_gguf_open(os.fsencode(p2), ctypes.byref(out)) == 0
    assert not mtg.lib().mtg_gguf_encoder(out)
    assert "enc.conv1.w: expected" in mtg.lib().mtg_gguf_error(out).decode()
    mtg.lib().mtg_gguf_close(out)
    # a missing adaptor tensor, an f16 projection
    p3 = str(tmp_path / "missing.gguf")
    gguf_writer.write_encoder(p3, syn, edit=lambda ts: [t for t in ts if t[0] != "adaptor.fc2.b"])
    enc = ctypes.c_void_p()
    assert mtg.lib().mtg_encoder_create_from_gguf(os.fsencode(p3), ctypes.byref(enc)) != 0
    assert "missing tensor adaptor.fc2.b" in mtg.lib().mtg_gguf_error(None).decode()

    def f16_k(ts):
        return [(n, 1, ne, np.zeros(ne[0] * ne[1], np.float16).tobytes()) if n == "enc.blk.0.attn_k.w" else (n, t, ne, dd)
                for n, t, ne, dd in ts]
    p4 = str(tmp_path / "f16k.gguf")
    gguf_writer.write_encoder(p4, syn, edit=f16_k)
    assert mtg.lib().mtg_encoder_create_from_gguf(os.fsencode(p4), ctypes.byref(enc)) != 0
    assert "must all be q8_0" in mtg.lib().mtg_gguf_error(None).decode()
    m.close()


@pytest.mark.parametrize("wtype", [mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K], ids=["f16", "f32", "q4_K"])
def test_encoder_f16_f32_and_q4k_round_trip(tmp_path, wtype):
    """An encoder whose matrices are f16 or f32 (the converter's f16 and default f32
    dtypes) or q4_K (cli quantize q4_k): the description carries the type and every tensor byte for
    byte; a q8_0 matrix among them is refused by name."""
    syn = mtg.SynthEncoder(seed=4, wtype=wtype, n_mels=16, n_frames=96, d_model=256, n_layers=2, n_heads=4,
                           ffn=512, merge=4, hidden=256)
    path = str(tmp_path / "enc.gguf")
    gguf_writer.write_encoder(path, syn)
    g = mtg.GgufModel(path, decoder=False)
    e = g.encoder().contents
    assert e.weight_type == wtype
    got, want = _enc_bytes(e, syn), _enc_bytes(syn.desc, syn)
    assert len(got) == len(want) and all(a == b for a, b in zip(got, want))
    g.close()

    def q8_v(ts):
        return [(n, 8, ne, bytes(mtg.lib().mtg_row_bytes(8, ne[0]) * ne[1])) if n == "enc.blk.1.attn_v.w"
                else (n, t, ne, dd) for n, t, ne, dd in ts]
    p2 = str(tmp_path / "mixed.gguf")
    gguf_writer.write_encoder(p2, syn, edit=q8_v)
    enc = ctypes.c_void_p()
    assert mtg.lib().mtg_encoder_create_from_gguf(os.fsencode(p2), ctypes.byref(enc)) != 0
    msg = mtg.lib().mtg_gguf_error(None).decode()
    assert "enc.blk.1.attn_v.w is q8_0" in msg, msg


def test_hand_assembled_file():
    """A GGUF v3 file assembled here byte by byte from the published layout (not by
    tests/gguf_writer.py): header, metadata of several types (a string array, a
    64-bit integer, general.alignment = 64), two tensor infos whose data offsets are
    relative to the 64-byte aligned data section. The loader must return each
    tensor's type, ne and bytes."""
    import tempfile

    def s(x):
        return struct.pack("<Q", len(x)) + x
    kv = [s(b"general.architecture") + struct.pack("<I", 8) + s(b"qwen3"),
          s(b"tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + s(b"a") + s(b"bc"),
          s(b"general.alignment") + struct.pack("<II", 4, 64),
          s(b"mtd.text.vocab_size") + struct.pack("<IQ", 10, 2)]
    q8 = bytes(range(68))                                # two q8_0 rows of 32: 2 x 34 bytes
    f32 = np.arange(3, dtype=np.float32).tobytes()
    infos = (s(b"w.q8") + struct.pack("<I2QIQ", 2, 32, 2, 8, 0) +
             s(b"v.f32") + struct.pack("<I1QIQ", 1, 3, 0, 128))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv)) + b"".join(kv) + infos
    data_start = (len(head) + 63) // 64 * 64
    blob = head + b"\0" * (data_start - len(head)) + q8 + b"\0" * (128 - len(q8)) + f32
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "hand.gguf")
        open(path, "wb").write(blob)
        g = mtg.GgufModel(path, decoder=False)
        assert mtg.lib().mtg_gguf_n_tensors(g.handle) == 2
        t, ne, raw = g.tensor("w.q8")
        assert (t, ne, raw) == (8, [32, 2, 1, 1], q8)
        t, ne, raw = g.tensor("v.f32")
        assert (t, ne, raw) == (0, [3, 1, 1, 1], f32)
        with pytest.raises(KeyError):
            g.tensor("absent")
        g.close()


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
def test_oracle_from_parsed_file_equals_oracle_from_model(model, tmp_path, kv_type):
    """The decoder description mtg_gguf_model builds from a file drives the oracle
    to the same hidden rows, logits and choices as the in-memory model it was
    written from (the device decoder from the same file is compared with this
    oracle in test_gpu_gguf.py)."""
    import oracle_py

    path = str(tmp_path / "m.gguf")
    gguf_writer.write_model(path, model)
    g = mtg.GgufModel(path)
    a = oracle_py.Oracle(model, 64, kv_type)
    b = oracle_py.Oracle(g, 64, kv_type)
    g.close()
    rng = np.random.default_rng(5)
    ids = rng.integers(0, model.hp.vocab, 20)
    rows = a.embed(ids)
    assert np.array_equal(b.embed(ids), rows)
    assert np.array_equal(b.prefill(rows).view(np.uint32), a.prefill(rows).view(np.uint32))
    tokens = rng.integers(0, model.hp.vocab, 5)
    ca, ma, ha, la = a.verify(tokens, want_hidden=True, want_logits=True)
    cb, mb, hb, lb = b.verify(tokens, want_hidden=True, want_logits=True)
    assert np.array_equal(hb.view(np.uint32), ha.view(np.uint32))
    assert np.array_equal(lb.view(np.uint32), la.view(np.uint32))
    assert np.array_equal(cb, ca) and mb == ma
    a.close()
    b.close()
