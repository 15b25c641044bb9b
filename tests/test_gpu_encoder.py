"""The Whisper encoder + audio adaptor on the device (csrc/encoder.hip; reference
WhisperEncoder::encode, src/whisper_encoder.cpp:103-209, AudioAdaptor::apply,
src/audio_adaptor.cpp:38-97) against the oracle: encoder rows and adaptor rows
bit-identical (the kernels keep the oracle's order of every reduction), at a
short chunk and at the full 3,000-frame chunk (1,500 rows) with 2 layers for
q8_0, f16, f32 and q4_K matrices, and for the whole 24-layer q8_0 encoder (also timed
and checked for determinism); and the whole path from mel frames to token ids
(encoder, adaptor, fused prompt, prefill, speculative steps) on both sides."""
import os

import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu


def _same(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g at %s"
                         % (what, int((got != ref).sum()), err.max(), np.unravel_index(err.argmax(), err.shape)))


WTYPES = [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K]
WT_IDS = ["q8_0", "f16", "f32", "q4_K"]


@pytest.mark.parametrize("wtype", WTYPES, ids=WT_IDS)
@pytest.mark.parametrize("n_frames,n_layers", [(160, 2), (333, 1)])
def test_encoder_and_adaptor_match_oracle(n_frames, n_layers, wtype):
    print("encoder vs oracle: %d frames, %d layers, weights %d" % (n_frames, n_layers, wtype), flush=True)
    syn = mtg.SynthEncoder(seed=3, wtype=wtype, n_frames=n_frames, n_layers=n_layers, ffn=2048)
    dev = mtg.Encoder(syn)
    orc = oracle_py.OracleEncoder(syn)
    mel = syn.mel(seed=4)
    rows = dev.encode(mel)
    _same(rows, orc.encode(mel), "encoder rows")
    for T in (syn.rows, syn.rows - 3, 4, 3):
        _same(dev.adapt(T), orc.adapt(T), "adaptor rows, T=%d" % T)
    # the adaptor on rows the caller hands over
    other = (mtg.normal(8, 0, syn.rows * 1024).reshape(syn.rows, 1024) * np.float32(0.7)).astype(np.float32)
    _same(dev.adapt(syn.rows, rows=other), orc.adapt(syn.rows, rows=other), "adaptor on host rows")
    dev.close()
    orc.close()


@pytest.mark.parametrize("wtype", WTYPES, ids=WT_IDS)
def test_full_chunk_two_layers_matches_oracle(wtype):
    """3,000 mel frames (1,500 rows, full width: d 1024, 16 heads, ffn 4096):
    the conv stem, attention over all 1,500 rows and the adaptor's 375 rows, for
    q8_0, f16 and q4_K matrices."""
    syn = mtg.SynthEncoder(seed=11, wtype=wtype, n_layers=2)
    dev = mtg.Encoder(syn)
    orc = oracle_py.OracleEncoder(syn)
    mel = syn.mel(seed=12)
    rows = dev.encode(mel)
    print("full chunk, 2 layers, weights %d: encode %.2f ms" % (wtype, dev.last_ms), flush=True)
    _same(rows, orc.encode(mel), "encoder rows")
    _same(dev.adapt(1500), orc.adapt(1500), "adaptor rows")
    _same(dev.adapt(552), orc.adapt(552), "adaptor rows of a trimmed chunk")
    dev.close()
    orc.close()


@pytest.mark.timeout(900)
def test_full_encoder_24_layers_matches_oracle():
    """The whole 24-layer encoder on the full 3,000-frame chunk and the adaptor's
    375 rows: bit-identical to the oracle, repeated encodes identical, timed."""
    syn = mtg.SynthEncoder(seed=21)
    dev = mtg.Encoder(syn)
    mel = syn.mel(seed=22)
    a = dev.encode(mel)
    ms = []
    for _ in range(3):
        b = dev.encode(mel)
        ms.append(dev.last_ms)
        _same(b, a, "repeated encode")
    ad = dev.adapt(1500)
    print("24-layer encoder, 3,000 frames -> 1,500 rows: %.2f ms (min of 3), adaptor %.3f ms"
          % (min(ms), dev.last_ms), flush=True)
    assert np.isfinite(a).all() and np.isfinite(ad).all()
    oracle_py.lib().orc_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    orc = oracle_py.OracleEncoder(syn)
    print("24-layer encoder: the oracle's encode", flush=True)
    _same(a, orc.encode(mel), "24-layer encoder rows")
    _same(ad, orc.adapt(1500), "adaptor rows after 24 layers")
    orc.close()
    # ln_post's output rows: (y - b) / w has mean 0 and variance 1 per row
    d = syn.desc
    w = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * 1024).from_address(d.ln_post_w))
    bb = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * 1024).from_address(d.ln_post_b))
    z = (a.astype(np.float64) - bb) / w
    assert np.abs(z.mean(axis=1)).max() < 1e-4 and np.abs(z.var(axis=1) - 1).max() < 1e-2
    dev.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("exec_mode", [mtg.EXEC_STEP_KERNEL, mtg.EXEC_GRAPH], ids=["step", "graph"])
def test_audio_to_tokens_matches_oracle(exec_mode):
    """The whole transcription path on both sides, from mel frames to token ids: a
    3,000-frame chunk through the encoder (2 layers) and the adaptor (375 rows), the
    prompt fused as the reference's fuse_embeds does (src/generate.cpp:113-178: the
    ids embedded, the k-th position holding the audio token id replaced by adaptor
    row k), the decoder's prefill of the fused rows (2 layers, hidden 1024), the first
    greedy id from the last row's logits, then 24 speculative steps with the n-gram
    drafter. Every intermediate and the committed ids are equal."""
    print("audio to tokens: exec %d" % exec_mode, flush=True)
    oracle_py.lib().orc_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    syn = mtg.SynthEncoder(seed=21, n_layers=2)
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=22, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    assert syn.hp.hidden == model.hp.hidden
    enc, oenc = mtg.Encoder(syn), oracle_py.OracleEncoder(syn)
    mel = syn.mel(seed=23)
    _same(enc.encode(mel), oenc.encode(mel), "encoder rows")
    a1, a0 = enc.adapt(syn.rows), oenc.adapt(syn.rows)
    _same(a1, a0, "adaptor rows")
    n_audio = a1.shape[0]
    rng = np.random.default_rng(24)
    audio_id = 4000
    prefix = rng.integers(0, audio_id, 12)
    suffix = rng.integers(0, audio_id, 40)
    ids = np.concatenate([prefix, np.full(n_audio, audio_id), suffix]).astype(np.int32)
    max_seq = len(ids) + 24 * 8 + 16
    dec = mtg.Decoder(model, max_seq, mtg.TYPE_F32)
    dec.set_exec(exec_mode)
    orc = oracle_py.Oracle(model, max_seq, mtg.TYPE_F32)

    def fuse(embed, audio):  # the k-th audio position takes audio row k
        rows = embed(ids).copy()
        rows[ids == audio_id] = audio
        return rows

    f1, f0 = fuse(dec.embed, a1), fuse(orc.embed, a0)
    _same(f1, f0, "fused prompt rows")
    h1, h0 = dec.prefill(f1), orc.prefill(f0)
    _same(h1, h0, "prefill hidden rows")
    l1, l0 = dec.logits(h1[-1:]), orc.logits(h0[-1:])
    _same(l1, l0, "logits of the last prompt row")
    first = int(np.argmax(l1[0]))
    ids1, st1 = dec.generate_from(first, 1 << 20, max_steps=24, max_draft=7)
    ids0, st0 = orc.generate_from(first, 1 << 20, max_steps=24, max_draft=7)
    assert ids1.tolist() == ids0.tolist()
    for f in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds"):
        assert getattr(st1, f) == getattr(st0, f), f
    print("audio to tokens: %d prompt rows (%d audio), %d ids" % (len(ids), n_audio, len(ids1)), flush=True)
    for x in (dec, orc, enc, oenc, model):
        x.close()
