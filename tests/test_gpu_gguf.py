"""Device decoders built from GGUF files (mtg_create_from_gguf) against decoders
built from the same seeded model in memory: prefill hidden rows, verify hidden
rows, logits and choices bit-identical, for q8_0, f16 and q4_K weights, and at
full size (28 layers, 151,936-row vocabulary) for a q8_0 file named and typed
the way the reference's converter writes one."""
import os
import time

import numpy as np
import pytest

import gguf_writer
import mtg

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), what


def _compare(model, path, kv_type, prefix, T):
    a = mtg.Decoder(model, prefix + 2 * T + 8, kv_type)
    b = mtg.Decoder.from_gguf(path, prefix + 2 * T + 8, kv_type)
    for f in ("hidden", "n_heads", "n_kv_heads", "head_dim", "intermediate", "n_layers", "vocab"):
        assert getattr(b.hp, f) == getattr(model.hp, f), f
    rng = np.random.default_rng(prefix + T)
    ids = rng.integers(0, model.hp.vocab, prefix)
    rows = a.embed(ids)
    _same(b.embed(ids), rows, "embedding rows")
    _same(b.prefill(rows), a.prefill(rows), "prefill hidden")
    for _ in range(2):
        tokens = rng.integers(0, model.hp.vocab, T)
        c0, m0, h0, l0 = a.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = b.verify(tokens, want_hidden=True, want_logits=True)
        _same(h1, h0, "verify hidden")
        _same(l1, l0, "logits")
        assert np.array_equal(c1, c0) and m1 == m0
    a.close()
    b.close()


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
@pytest.mark.parametrize("wtype", [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_Q4_K], ids=["q8_0", "f16", "q4_K"])
def test_decoder_from_gguf_equals_decoder_from_model(wtype, kv_type, tmp_path):
    print("decoder from a GGUF file: weight type %d kv %d" % (wtype, kv_type), flush=True)
    model = mtg.SynthModel(wtype, seed=21, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    path = str(tmp_path / "m.gguf")
    gguf_writer.write_model(path, model)
    _compare(model, path, kv_type, 40, 8)
    model.close()


def test_full_size_q8_0_file(tmp_path):
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=0, std=0.02, gain_jitter=0.0)
    path = str(tmp_path / "qwen3-0.6b-q8_0.gguf")
    t0 = time.perf_counter()
    gguf_writer.write_model(path, model)
    t1 = time.perf_counter()
    print("full-size q8_0 GGUF: %.0f MB written in %.1f s" % (os.path.getsize(path) / 1e6, t1 - t0), flush=True)
    _compare(model, path, mtg.TYPE_F32, 100, 8)
    model.close()


def test_encoder_from_gguf_equals_encoder_from_model(tmp_path):
    syn = mtg.SynthEncoder(seed=31, n_frames=160, n_layers=2, ffn=2048)
    path = str(tmp_path / "enc.gguf")
    gguf_writer.write_encoder(path, syn)
    a = mtg.Encoder(syn)
    b = mtg.Encoder.from_gguf(path)
    mel = syn.mel(seed=32)
    _same(b.encode(mel), a.encode(mel), "encoder rows")
    _same(b.adapt(80), a.adapt(80), "adaptor rows")
    a.close()
    b.close()
