"""The drop-in loader snippet of the repository's integration guide reads the
tensors the reference's loader reads, in the field order of mtg_layer_tensors.

Expected names (data, cited): qwen3_load_layer reads prefix + ".blk.<i>." + one of
the eleven names below with prefix "qwen3" (src/qwen3.cpp:33-56), and
Qwen3Decoder::load reads "qwen3.output_norm.weight" and "token_embd.weight"
(src/qwen3_decoder.cpp:53-57); the converter writes the same names
(scripts/convert_moss_transcribe_to_gguf.py:242-259). When the reference tree is
present the names are also extracted from its loader source."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"

# qwen3_load_layer's names in the order of Qwen3Layer / mtg_layer_tensors
LAYER_NAMES = ["attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
               "attn_o.weight", "attn_q_norm.weight", "attn_k_norm.weight", "ffn_norm.weight",
               "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"]
GLOBAL_NAMES = {"token_embd.weight", "qwen3.output_norm.weight"}


def _snippet():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    for b in blocks:
        if "mtg_desc_from_loader" in b:
            return b
    raise AssertionError("the integration guide has no loader snippet")


def _struct_fields():
    h = open(os.path.join(ROOT, "include", "mtg_verify.h")).read()
    body = re.search(r"typedef struct mtg_layer_tensors \{(.*?)\} mtg_layer_tensors;", h, re.S).group(1)
    return re.findall(r"\*\s*(\w+);", body)


def test_layer_names_and_order():
    s = _snippet()
    init = re.search(r"L\[i\] = \{(.*?)\};", s, re.S).group(1)
    names = re.findall(r'T\("([^"]+)"\)', init)
    assert names == LAYER_NAMES
    # the initializer follows the struct's field order: field f <- the name of f
    fields = _struct_fields()
    assert len(fields) == len(names)
    for f, n in zip(fields, names):
        stem = n[: -len(".weight")]
        assert f == stem or f == "attn_" + stem[len("attn_"):], (f, n)
    assert '"qwen3.blk." + std::to_string(i) + "."' in s


def test_global_names_and_null_checks():
    s = _snippet()
    names = set(re.findall(r'bytes\("([^"]+)"\)', s))
    assert names == GLOBAL_NAMES
    # every lookup is checked: a missing tensor fails the helper, not ggml_nbytes
    assert re.search(r"if \(!t\)", s) and "return false" in s
    assert "mtg_desc_from_loader(m, layers, copies, &desc) &&" in s


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="reference tree not present")
def test_names_match_the_reference_loader_source():
    src = open(os.path.join(REF, "src", "qwen3.cpp")).read()
    body = src[src.index("bool qwen3_load_layer(const ModelLoader& m, const std::string& prefix"):]
    body = body[: body.index("return ok;")]
    assert re.findall(r'get\("([^"]+)"', body) == LAYER_NAMES
    dec = open(os.path.join(REF, "src", "qwen3_decoder.cpp")).read()
    for n in GLOBAL_NAMES:
        assert 'm.tensor("%s")' % n in dec
