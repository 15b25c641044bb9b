"""The C-ABI boundary on the CPU: libmtg.so loads, exports every function that
include/mtg_verify.h declares, the Python binding's struct layouts match the C
ones, host-only entry points work without a GPU, and a missing library fails
loudly instead of falling back to anything."""
import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import mtg
import oracle_py

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtg_verify.h")


def _declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"typedef[^;]*;", "", text, flags=re.S)
    names = set(re.findall(r"\b(mtg_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    names = _declared_functions(HEADER)
    assert len(names) >= 39
    lib = ctypes.CDLL(mtg.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding covers exactly the declared set
    assert sorted(mtg.SIGNATURES) == names


def test_oracle_exports_its_header():
    names = sorted(set(re.findall(r"\b(orc_\w+)\s*\(", re.sub(r"typedef[^;]*;", "",
                   open(os.path.join(ROOT, "oracle", "oracle.h")).read(), flags=re.S))))
    lib = ctypes.CDLL(oracle_py.LIB_PATH)
    assert [n for n in names if not hasattr(lib, n)] == []


def test_abi_version():
    assert mtg.lib().mtg_abi_version() == 1


STRUCTS = {
    "mtg_hparams": (mtg.Hparams, ["hidden", "n_heads", "n_kv_heads", "head_dim", "intermediate",
                                  "n_layers", "vocab", "rope_base", "rms_eps"]),
    "mtg_layer_tensors": (mtg.LayerTensors, ["attn_norm", "attn_q", "ffn_down"]),
    "mtg_model_desc": (mtg.ModelDesc, ["hp", "weight_type", "token_embd", "output_norm", "layers"]),
    "mtg_gen_stats": (mtg.GenStats, ["target_calls", "rewinds", "prefill_seconds", "draft_seconds",
                                     "stop_reason", "next_seed"]),
    "mtg_stream_drafter": (mtg.StreamDrafter, ["prompt", "n_prompt", "stream", "period"]),
    "mtg_target": (mtg.Target, ["self", "verify", "past", "max_seq", "vocab"]),
}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layouts_match_the_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "%s"' % HEADER, "int main(void){"]
    for cname, (_, fields) in STRUCTS.items():
        lines.append('printf("%s %%zu\\n", sizeof(%s));' % (cname, cname))
        for f in fields:
            lines.append('printf("%s.%s %%zu\\n", offsetof(%s, %s));' % (cname, f, cname, f))
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout
    got = dict(l.split() for l in out.strip().splitlines())
    for cname, (py, fields) in STRUCTS.items():
        assert int(got[cname]) == ctypes.sizeof(py), cname
        for f in fields:
            assert int(got["%s.%s" % (cname, f)]) == getattr(py, f).offset, (cname, f)


def test_host_entry_points_need_no_gpu():
    L = mtg.lib()
    # f16 conversion, quantizers and the normal stream are host code
    assert L.mtg_f16_to_f32(0x3C00) == 1.0 and L.mtg_f32_to_f16(-2.0) == 0xC000
    assert L.mtg_row_bytes(mtg.TYPE_Q8_0, 1024) == 32 * 34
    assert L.mtg_row_bytes(mtg.TYPE_Q4_K, 1024) == 4 * 144
    assert L.mtg_row_bytes(mtg.TYPE_F16, 1024) == 2048
    a, b = mtg.normal(7, 0, 1000), mtg.normal(7, 500, 500)
    assert np.array_equal(a[500:], b)  # addressable stream
    assert abs(a.mean()) < 0.1 and abs(a.std() - 1) < 0.1


def test_q8_0_weight_quantizer_round_trip():
    """GGUF converter rule: d = amax/127 stored f16, codes = round-half-away(x/d)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(64 * 32) * 0.02).astype(np.float32)
    raw = np.empty(64 * 34, np.uint8)
    mtg.lib().mtg_quantize_q8_0_weight(mtg.ptr(x), x.size, mtg.ptr(raw))
    blk = raw.view(oracle_py.Q8_BLOCK)
    d = (np.abs(x.reshape(-1, 32)).max(axis=1) / np.float32(127)).astype(np.float32)
    assert np.array_equal(blk["d"], d.astype(np.float16).view(np.uint16))
    idv = (np.float32(1) / d).astype(np.float32)
    v = (x.reshape(-1, 32) * idv[:, None]).astype(np.float32)
    want = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    assert np.array_equal(blk["qs"], want)
    back = np.empty_like(x)
    mtg.lib().mtg_dequantize(mtg.TYPE_Q8_0, mtg.ptr(raw), x.size, mtg.ptr(back))
    assert np.abs(back - x).max() <= np.abs(x).max() / 127


def test_missing_library_raises(monkeypatch):
    monkeypatch.setattr(mtg, "_lib", None)
    monkeypatch.setattr(mtg, "LIB_PATH", os.path.join(ROOT, "no-such-dir", "libmtg.so"))
    with pytest.raises(FileNotFoundError):
        mtg.lib()


def test_entry_points_reject_null_context():
    L = mtg.lib()
    assert L.mtg_rewind(None, 0) == mtg.ERR_INVALID
    assert L.mtg_verify(None, None, 1, None, 0, 1.0, None, None, None, None) == mtg.ERR_INVALID
    assert L.mtg_past_len(None) == 0
    assert L.mtg_create(None, 16, mtg.TYPE_F32, None) == mtg.ERR_INVALID
