"""CPU tests of the GGUF reader (aspida_gguf_*, aspida_amd.gguf) on files
written here: descriptors, byte sizes and data against the closed forms of
Checked_Byte_Size (src/llm/llm_gguf.adb:238-258), the alignment rule
(433-455, 500-506), every rejection the reference makes (bad magic, absurd
counts, over-long strings, more than 4 dims, data past the end of the file),
and the Q4_K_M mix (tools/probes/requantize.adb:103-113)."""
import numpy as np
import pytest

import aspida_amd as aa
from aspida_amd import gguf, synth
import gguf_writer as gw

# GGML type codes (To_GGML_Type, llm_gguf.adb:266-291)
F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16, IQ2_XXS = 0, 1, 8, 10, 11, 12, 13, 14, 30, 16
KIND = {Q4_K: aa.Q4_K, Q6_K: aa.Q6_K, Q5_K: aa.Q5_K, Q3_K: aa.Q3_K, Q2_K: aa.Q2_K, Q8_0: aa.Q8_0}


def _model(gen):
    """A small Q4_K_M-shaped model: one layer, head, embeddings, a norm."""
    def kq(kind_code, out, inp):
        return synth.weight_np(KIND[kind_code], out, inp, gen).tobytes()
    return [
        ("token_embd.weight", [512, 64], F32, gen.standard_normal(512 * 64).astype(np.float32).tobytes()),
        ("blk.0.attn_norm.weight", [512], F32, np.ones(512, np.float32).tobytes()),
        ("blk.0.attn_q.weight", [512, 256], Q4_K, kq(Q4_K, 256, 512)),
        ("blk.0.attn_v.weight", [512, 64], Q6_K, kq(Q6_K, 64, 512)),
        ("blk.0.ffn_up.weight", [512, 130], Q4_K, kq(Q4_K, 130, 512)),
        ("blk.0.ffn_down.weight", [768, 512], Q6_K, kq(Q6_K, 512, 768)),
        ("blk.0.ffn_gate.weight", [512, 96], Q5_K, kq(Q5_K, 96, 512)),
        ("blk.0.extra_q3.weight", [256, 10], Q3_K, kq(Q3_K, 10, 256)),
        ("blk.0.extra_q2.weight", [256, 12], Q2_K, kq(Q2_K, 12, 256)),
        ("blk.0.extra_q8.weight", [256, 7], Q8_0, kq(Q8_0, 7, 256)),
        ("blk.0.f16.weight", [33], F16, np.arange(33, dtype=np.float16).tobytes()),
        ("blk.0.bf16.weight", [5, 3], BF16, bytes(30)),
        ("output.weight", [512, 300], Q6_K, kq(Q6_K, 300, 512)),
    ]


META = [("general.architecture", "str", "llama"), ("general.alignment", "u32", 64),
        ("llama.block_count", "u32", 1), ("llama.rope.freq_base", "f32", 500000.0),
        ("tokenizer.ggml.tokens", "arr", ("str", ["<s>", "a,b", "[x]"])),
        ("tokenizer.ggml.scores", "arr", ("f32", [0.0, -1.5, 2.25])), ("general.flag", "bool", 1),
        ("general.tags", "arr", ("str", ["x", "y"])), ("general.grid", "arr", ("arr", [("i32", [1, -2]), ("u8", [])])),
        ("general.big", "u64", 1 << 40), ("general.neg", "i64", -7), ("general.d", "f64", 0.125)]


def _expected_bytes(gt, n):
    per = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110),
           Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
    blk, size = per.get(gt, (1, 4))
    return (n + blk - 1) // blk * size


def test_model_file_layout(tmp_path):
    gen = synth.rng(5)
    tensors = _model(gen)
    path = tmp_path / "m.gguf"
    start, offs = gw.write(path, tensors, META, alignment=64)
    with gguf.GGUFFile(path) as g:
        assert g.version == 3 and g.alignment == 64 and g.data_start == start
        assert [t["name"] for t in g.tensors] == [t[0] for t in tensors]
        for (name, dims, gt, data), o in zip(tensors, offs):
            t = g.by_name[name]
            assert t["dims"] == dims and t["ggml_type"] == gt
            assert t["kind"] == KIND.get(gt, -1)
            assert t["bytes"] == _expected_bytes(gt, int(np.prod(dims))) == len(data)
            assert t["offset"] == start + o and t["offset"] % 64 == 0
            assert bytes(g.data(name)) == data
        assert g.meta("general.architecture") == "llama"
        assert g.meta("llama.block_count") == "1"
        assert float(g.meta("llama.rope.freq_base")) == 500000.0
        assert g.meta("tokenizer.ggml.tokens") == "[array: 3]"          # the reference's token list form
        assert g.meta("tokenizer.ggml.scores") == "[0, -1.5, 2.25]"
        assert g.meta("general.tags") == "[x, y]" and g.meta("general.grid") == "[[1, -2], []]"
        assert g.meta("general.flag") == "true" and g.meta("general.big") == str(1 << 40)
        assert g.meta("general.neg") == "-7" and float(g.meta("general.d")) == 0.125
        assert g.meta("missing.key") is None
        raw, kind, in_dim, out_dim = g.weight("blk.0.ffn_down.weight")
        assert (kind, in_dim, out_dim) == (aa.Q6_K, 768, 512)
        with pytest.raises(ValueError):
            g.weight("token_embd.weight")          # F32: not a kind the kernels run
        assert g.check_q4_k_m() == ["blk.0.ffn_gate.weight", "blk.0.extra_q3.weight",
                                    "blk.0.extra_q2.weight", "blk.0.extra_q8.weight"]


def test_read_entry_point_copies_the_bytes(tmp_path):
    gen = synth.rng(6)
    data = synth.weight_np(aa.Q4_K, 3, 256, gen).tobytes()
    path = tmp_path / "r.gguf"
    gw.write(path, [("w", [256, 3], Q4_K, data)])
    lib = gguf._bind(aa.load())
    h = lib.aspida_gguf_open(str(path).encode())
    assert h
    buf = np.zeros(len(data), np.uint8)
    assert lib.aspida_gguf_read(h, 0, buf.ctypes.data, buf.size) == len(data)
    assert buf.tobytes() == data
    assert lib.aspida_gguf_read(h, 0, buf.ctypes.data, buf.size - 1) < 0      # too small a buffer
    assert lib.aspida_gguf_read(h, 1, buf.ctypes.data, buf.size) < 0          # no such tensor
    assert lib.aspida_gguf_find(h, b"w") == 0 and lib.aspida_gguf_find(h, b"v") == -1
    lib.aspida_gguf_close(h)


def test_reference_byte_size_rules(tmp_path):
    """Checked_Byte_Size: partial final blocks round up; types it does not list
    (here IQ2_XXS) count 4 bytes per element and get no kind."""
    path = tmp_path / "s.gguf"
    gw.write(path, [("q8", [40], Q8_0, bytes(68)), ("q4k", [300], Q4_K, bytes(288)),
                    ("iq", [10], IQ2_XXS, bytes(40))])
    with gguf.GGUFFile(path) as g:
        assert g.by_name["q8"]["bytes"] == 68 and g.by_name["q4k"]["bytes"] == 288
        assert g.by_name["iq"]["bytes"] == 40 and g.by_name["iq"]["kind"] == -1


@pytest.mark.parametrize("alignment", [0, 48, 131072])
def test_invalid_alignment_keeps_32(tmp_path, alignment):
    path = tmp_path / "a.gguf"
    start, offs = gw.write(path, [("w", [256, 1], Q4_K, bytes(144)), ("v", [256, 1], Q4_K, bytes(144))],
                           [("general.alignment", "u32", alignment)], alignment=32)
    with gguf.GGUFFile(path) as g:
        assert g.alignment == 32 and g.data_start == start
        assert g.by_name["v"]["offset"] == start + offs[1]


def test_version_two_and_empty(tmp_path):
    path = tmp_path / "v2.gguf"
    gw.write(path, [], [("k", "str", "v")], version=2)
    with gguf.GGUFFile(path) as g:
        assert g.version == 2 and g.tensors == [] and g.meta("k") == "v"


def _bad(tmp_path, **kw):
    path = tmp_path / "bad.gguf"
    gw.write(path, **kw)
    with pytest.raises(ValueError) as e:
        gguf.GGUFFile(path)
    return str(e.value)


def test_rejections(tmp_path):
    w = [("w", [256, 2], Q4_K, bytes(288))]
    assert "magic" in _bad(tmp_path, tensors=w, magic=b"GGUX")
    assert "cap" in _bad(tmp_path, tensors=w, n_tensors=16385)
    assert "cap" in _bad(tmp_path, tensors=w, meta=[("k", "u8", 1)], n_meta=20000)
    assert "1 MiB" in _bad(tmp_path, tensors=[], meta=[("k", "str", "x" * (1048576 + 1))])
    assert "dims" in _bad(tmp_path, tensors=[("t", [1, 1, 1, 1, 1], F32, bytes(4))])
    assert "metadata value type" in _bad(tmp_path, tensors=[], meta=[("k", 13, b"\0" * 8)])
    deep = ("u8", [1])
    for _ in range(8):
        deep = ("arr", [deep])
    assert "nested" in _bad(tmp_path, tensors=[], meta=[("k", "arr", deep)])
    # a descriptor claiming more data than the file holds
    path = tmp_path / "short.gguf"
    gw.write(path, w)
    with open(path, "r+b") as f:
        f.truncate(path.stat().st_size - 1)
    with pytest.raises(ValueError, match="past the end"):
        gguf.GGUFFile(path)
    # a header cut off in the middle
    path2 = tmp_path / "cut.gguf"
    gw.write(path2, w, META)
    with open(path2, "r+b") as f:
        f.truncate(40)
    with pytest.raises(ValueError, match="short read"):
        gguf.GGUFFile(path2)
    with pytest.raises(ValueError, match="cannot open"):
        gguf.GGUFFile(tmp_path / "missing.gguf")


def test_q4_k_m_mix_names():
    assert gguf.q4_k_m_kind("output.weight") == aa.Q6_K
    assert gguf.q4_k_m_kind("blk.7.attn_v.weight") == aa.Q6_K
    assert gguf.q4_k_m_kind("blk.7.ffn_down.weight") == aa.Q6_K
    assert gguf.q4_k_m_kind("blk.7.attn_output.weight") == aa.Q4_K    # not the head
    assert gguf.q4_k_m_kind("blk.7.attn_q.weight") == aa.Q4_K
