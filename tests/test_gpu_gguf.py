"""Device decoders built from GGUF files (mtg_create_from_gguf) against the oracle
built from the parsed file (mtg_gguf_model's description of the same file): the
embedding rows, the prefill's hidden rows and KV cache, the verify steps' hidden
rows, logits and choices, bit for bit, for q8_0, f16 and q4_K weights and both KV
types, and at full size (28 layers, 151,936-row vocabulary) for a q8_0 file named
and typed the way the reference's converter writes one
(src/model_loader.cpp:21-169, scripts/convert_moss_transcribe_to_gguf.py:242-259).
The encoder read from a file is compared with the oracle's encoder over the same
seeded model."""
import os
import time

import numpy as np
import pytest

import gguf_writer
import mtg
import oracle_py

pytestmark = pytest.mark.gpu


def _same(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g"
                         % (what, int((got != ref).sum()), err.max()))


def _threads():
    oracle_py.lib().orc_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))


def _compare_with_oracle(path, kv_type, prefix, T, hp_ref):
    """The decoder mtg_create_from_gguf builds from `path` against the oracle
    built from mtg_gguf_model's description of the same file."""
    g = mtg.GgufModel(path)
    for f in ("hidden", "n_heads", "n_kv_heads", "head_dim", "intermediate", "n_layers", "vocab"):
        assert getattr(g.hp, f) == getattr(hp_ref, f), f
    max_seq = prefix + 2 * T + 8
    orc = oracle_py.Oracle(g, max_seq, kv_type)
    g.close()  # the oracle holds copies of the tensors
    dec = mtg.Decoder.from_gguf(path, max_seq, kv_type)
    rng = np.random.default_rng(prefix + T)
    ids = rng.integers(0, hp_ref.vocab, prefix)
    rows = orc.embed(ids)
    _same(dec.embed(ids), rows, "embedding rows")
    _same(dec.prefill(rows), orc.prefill(rows), "prefill hidden")
    k0, v0 = orc.kv_read(prefix)
    k1, v1 = dec.kv_read(prefix)
    _same(k1, k0, "K cache after the prefill")
    _same(v1, v0, "V cache after the prefill")
    for step in range(2):
        tokens = rng.integers(0, hp_ref.vocab, T)
        hist = rng.integers(0, hp_ref.vocab, 40) if step else ()
        pen = 1.3 if step else 1.0
        c0, m0, h0, l0 = orc.verify(tokens, history=hist, penalty=pen, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, history=hist, penalty=pen, want_hidden=True, want_logits=True)
        _same(h1, h0, "verify hidden, step %d" % step)
        _same(l1, l0, "logits, step %d" % step)
        assert np.array_equal(c1, c0) and m1 == m0, "choices, step %d" % step
    assert dec.past_len == orc.past_len == prefix + 2 * T
    dec.close()
    orc.close()


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
@pytest.mark.parametrize("wtype", [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K], ids=["q8_0", "f16", "f32", "q4_K"])
def test_decoder_from_gguf_matches_oracle(wtype, kv_type, tmp_path):
    print("decoder from a GGUF file against the oracle: weight type %d kv %d" % (wtype, kv_type), flush=True)
    _threads()
    model = mtg.SynthModel(wtype, seed=21, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    path = str(tmp_path / "m.gguf")
    gguf_writer.write_model(path, model)
    hp = model.hp
    model.close()  # nothing below reads the in-memory model
    _compare_with_oracle(path, kv_type, 40, 8, hp)


def test_decoder_from_gguf_f16_norms_matches_oracle(tmp_path):
    """Norm gains stored as f16 (the converter's f16 output type) are widened to
    f32 by the loader; the oracle reads the same widened description."""
    _threads()
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=22, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    path = str(tmp_path / "m16.gguf")
    gguf_writer.write_model(path, model, f16_norms=True)
    hp = model.hp
    model.close()
    _compare_with_oracle(path, mtg.TYPE_F32, 33, 4, hp)


def test_full_size_q8_0_file_matches_oracle(tmp_path):
    print("full-size q8_0 GGUF against the oracle", flush=True)
    _threads()
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=0, std=0.02, gain_jitter=0.0)
    path = str(tmp_path / "qwen3-0.6b-q8_0.gguf")
    t0 = time.perf_counter()
    gguf_writer.write_model(path, model)
    t1 = time.perf_counter()
    print("full-size q8_0 GGUF: %.0f MB written in %.1f s" % (os.path.getsize(path) / 1e6, t1 - t0), flush=True)
    hp = model.hp
    assert (hp.n_layers, hp.hidden, hp.vocab) == (28, 1024, 151936)
    model.close()
    _compare_with_oracle(path, mtg.TYPE_F32, 100, 8, hp)


class _ParsedEncoder:
    """mtg_gguf_encoder's description of a file, in the form OracleEncoder reads."""

    def __init__(self, g):
        self.desc = g.encoder().contents
        self.hp = self.desc.hp
        self.rows = (self.hp.n_frames - 1) // 2 + 1


@pytest.mark.parametrize("wtype", [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K], ids=["q8_0", "f16", "f32", "q4_K"])
def test_encoder_from_gguf_matches_oracle(tmp_path, wtype):
    syn = mtg.SynthEncoder(seed=31, wtype=wtype, n_frames=160, n_layers=2, ffn=2048)
    path = str(tmp_path / "enc.gguf")
    gguf_writer.write_encoder(path, syn)
    mel = syn.mel(seed=32)
    del syn
    g = mtg.GgufModel(path, decoder=False)
    ref = oracle_py.OracleEncoder(_ParsedEncoder(g))  # copies the tensors
    g.close()
    b = mtg.Encoder.from_gguf(path)
    _same(b.encode(mel), ref.encode(mel), "encoder rows")
    _same(b.adapt(80), ref.adapt(80), "adaptor rows")
    b.close()
    ref.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("wtype", [mtg.TYPE_Q8_0, mtg.TYPE_F32], ids=["q8_0", "f32"])
def test_one_file_audio_to_tokens_matches_oracle(tmp_path, wtype):
    """One GGUF file holding the decoder and the encoder + adaptor (as the
    reference's converter writes them, q8_0 or its default f32), read once by the
    device (mtg_create_from_gguf, mtg_encoder_create_from_gguf) and once parsed for
    the oracle: a 3,000-frame chunk through the encoder and the adaptor, the prompt
    fused as fuse_embeds does (src/generate.cpp:113-178), the prefill and 16
    speculative steps give the same rows and ids on both sides."""
    print("one file, audio to tokens: weights %d" % wtype, flush=True)
    _threads()
    syn = mtg.SynthEncoder(seed=41, wtype=wtype, n_layers=2)
    model = mtg.SynthModel(wtype, seed=42, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    path = str(tmp_path / "moss.gguf")
    gguf_writer.write_encoder(path, syn, model=model)
    mel = syn.mel(seed=43)
    model.close()
    del syn, model
    g = mtg.GgufModel(path)
    oenc = oracle_py.OracleEncoder(_ParsedEncoder(g))  # copies the tensors
    rng = np.random.default_rng(44)
    audio_id = 4000
    n_audio = oenc.rows // oenc.hp.merge
    ids = np.concatenate([rng.integers(0, audio_id, 9), np.full(n_audio, audio_id),
                          rng.integers(0, audio_id, 30)]).astype(np.int32)
    max_seq = len(ids) + 16 * 8 + 16
    orc = oracle_py.Oracle(g, max_seq, mtg.TYPE_F32)
    g.close()
    enc = mtg.Encoder.from_gguf(path)
    dec = mtg.Decoder.from_gguf(path, max_seq, mtg.TYPE_F32)
    _same(enc.encode(mel), oenc.encode(mel), "encoder rows")
    a1, a0 = enc.adapt(oenc.rows), oenc.adapt(oenc.rows)
    _same(a1, a0, "adaptor rows")
    assert a1.shape[0] == n_audio

    def fuse(embed, audio):
        rows = embed(ids).copy()
        rows[ids == audio_id] = audio
        return rows

    h1, h0 = dec.prefill(fuse(dec.embed, a1)), orc.prefill(fuse(orc.embed, a0))
    _same(h1, h0, "prefill hidden rows")
    first = int(np.argmax(dec.logits(h1[-1:])[0]))
    assert first == int(np.argmax(orc.logits(h0[-1:])[0]))
    ids1, st1 = dec.generate_from(first, 1 << 20, max_steps=16, max_draft=7)
    ids0, st0 = orc.generate_from(first, 1 << 20, max_steps=16, max_draft=7)
    assert ids1.tolist() == ids0.tolist()
    for f in ("target_calls", "proposed", "accepted", "rewinds"):
        assert getattr(st1, f) == getattr(st0, f), f
    print("one file, audio to tokens: %d prompt rows (%d audio), %d ids" % (len(ids), n_audio, len(ids1)), flush=True)
    for x in (dec, orc, enc, oenc):
        x.close()
