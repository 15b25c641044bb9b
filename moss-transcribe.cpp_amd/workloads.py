"""The benchmark workloads of the speculative verify step, as synthetic data.

Five configurations of the Qwen3-0.6B decoder (28 layers, hidden 1024, 16 / 8
heads, 151,936-row tied vocabulary): weights seeded N(0, 0.02) (seed 0), the
prompt built from blocks of 375 audio rows (N(0, 1) rows scaled to the RMS of the
token embeddings, the shape of the reference's fused audio prefix) followed by
random text ids, and a 37-token periodic draft stream for the n-gram drafter.
Used by bench.py and by the full-size tests.
"""
import numpy as np

import mtg

# (weight type, kv type, audio blocks, text ids, K rows, decode steps)
WORKLOADS = {
    1: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F32, blocks=0, text=512, K=4, steps=1),
    2: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F32, blocks=4, text=100, K=8, steps=256),
    3: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F16, blocks=10, text=250, K=16, steps=128),
    4: dict(wtype=mtg.TYPE_F16, kv=mtg.TYPE_F16, blocks=20, text=500, K=8, steps=128),
    5: dict(wtype=mtg.TYPE_Q4_K, kv=mtg.TYPE_F16, blocks=43, text=259, K=16, steps=64),
}
AUDIO_ROWS = 375
STREAM_PERIOD = 37
WNAME = {mtg.TYPE_Q8_0: "q8_0", mtg.TYPE_F16: "f16", mtg.TYPE_F32: "f32", mtg.TYPE_Q4_K: "q4_K"}


def prompt_rows(cfg):
    return cfg["blocks"] * AUDIO_ROWS + cfg["text"]


def build_prompt(model, embed, cfg):
    """Fused prompt rows (audio blocks, then the text ids' embeddings), the text
    ids and one period of the draft stream. embed(ids) -> rows (any decoder's)."""
    hp = model.hp
    rng = np.random.default_rng(1)
    text = rng.integers(0, hp.vocab, cfg["text"]).astype(np.int32)
    sample = embed(np.arange(0, hp.vocab, max(1, hp.vocab // 2048))[:2048])
    rms = float(np.sqrt((sample.astype(np.float64) ** 2).mean()))
    n_audio = cfg["blocks"] * AUDIO_ROWS
    audio = mtg.normal(1, 0, n_audio * hp.hidden).reshape(n_audio, hp.hidden) * np.float32(rms)
    rows = np.concatenate([audio, embed(text)]) if n_audio else embed(text)
    stream = np.random.default_rng(2).integers(0, hp.vocab, STREAM_PERIOD).astype(np.int32)
    return rows.astype(np.float32), text, stream
