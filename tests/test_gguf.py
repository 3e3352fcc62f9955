"""Packed GGUF loader (barq_rocm_gguf_*): the reference reader's rules
(barq_core/src/gguf.rs:250-413) on files written here, without a GPU."""
import os

import numpy as np
import pytest

import barq_rocm._lib as L
from barq_rocm import synth
from barq_rocm.gguf import GgufFile
import gguf_writer as W


def _tensors():
    rng = np.random.default_rng(5)
    return [
        ("token_embd.weight", [8, 3], 0, rng.standard_normal(24).astype(np.float32).tobytes()),
        ("norm.weight", [16], 1, rng.standard_normal(16).astype(np.float16).tobytes()),
        ("blk.0.attn_q.weight", [64, 2], 2, synth.gen_weights(L.Q4_0, 4, 32, 11).tobytes()),
        ("blk.0.attn_k.weight", [32, 3], 8, synth.gen_weights(L.Q8_0, 3, 32, 12).tobytes()),
        ("blk.0.ffn_up.weight", [256, 3], 12, synth.gen_q4_k(3, 256, 13).tobytes()),
        ("blk.0.ffn_down.weight", [512, 2], 14, synth.gen_q6_k(2, 512, 14).tobytes()),
        ("blk.0.iq.weight", [256, 1], 16, bytes(136)),   # IQ4_KS: accepted, not sized (the reference cannot load it)
    ]


KVS = [
    ("general.architecture", W.STRING, "llama"),
    ("general.name", W.STRING, "tést ✓"),
    ("llama.block_count", W.U32, 32),
    ("llama.context_length", W.U64, 8192),
    ("llama.rope.freq_base", W.F32, 500000.0),
    ("llama.attention.layer_norm_rms_epsilon", W.F32, 1e-5),
    ("u8", W.U8, 255), ("i8", W.I8, -128), ("u16", W.U16, 65535), ("i16", W.I16, -32768),
    ("i32", W.I32, -7), ("i64", W.I64, -(1 << 40)), ("f64", W.F64, 0.25), ("flag", W.BOOL, True),
    ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<s>", "</s>", "é"])),
    ("tokenizer.ggml.scores", W.ARRAY, (W.F32, [0.0, -1.5, 2.0, 3.0])),
    ("nested", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.STRING, ["a"])])),
    ("dup", W.U32, 1), ("dup", W.U32, 2),   # HashMap::insert: the last one stays
]


@pytest.fixture(scope="module")
def gfile(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gguf") / "model.gguf")
    data_offset, offsets = W.write(p, KVS, _tensors())
    return p, data_offset, offsets


def test_header_kv_and_tensor_infos(gfile):
    p, data_offset, offsets = gfile
    ts = _tensors()
    with GgufFile(p) as g:
        info = g.info()
        assert info == dict(version=3, n_tensors=len(ts), n_kv=len(KVS), alignment=32, data_offset=data_offset)
        assert g.kv_string("general.architecture") == "llama"
        assert g.kv_string("general.name") == "tést ✓"
        assert g.kv_int("llama.block_count") == 32 and g.kv_int("llama.context_length") == 8192
        assert g.kv_number("llama.rope.freq_base") == 500000.0
        assert g.kv_number("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        assert (g.kv_int("u8"), g.kv_int("i8"), g.kv_int("u16"), g.kv_int("i16")) == (255, -128, 65535, -32768)
        assert (g.kv_int("i32"), g.kv_int("i64"), g.kv_number("f64"), g.kv_int("flag")) == (-7, -(1 << 40), 0.25, 1)
        assert g.kv_type("tokenizer.ggml.tokens") == (W.ARRAY, W.STRING, 3)
        assert g.kv_type("tokenizer.ggml.scores") == (W.ARRAY, W.F32, 4)
        assert g.kv_type("nested") == (W.ARRAY, W.ARRAY, 2)
        assert g.kv_int("dup") == 2
        for i, ((name, dims, tid, raw), off) in enumerate(zip(ts, offsets)):
            t = g.tensor(i)
            assert t["name"] == name and t["type"] == tid and t["n_dims"] == len(dims)
            assert t["dims"][:len(dims)] == dims and t["offset"] == off
            if tid == 16:
                assert t["nbytes"] == 0 and t["data"] is None
            else:
                # the packed bytes at data_offset + offset (gguf.rs:428-431), untouched
                assert t["nbytes"] == len(raw) and t["data"].tobytes() == raw
            assert g.find(name) == i


def test_errors_follow_the_reference(tmp_path):
    p = str(tmp_path / "x.gguf")
    lib = L.lib()

    def open_rc(path):
        import ctypes
        h = ctypes.c_void_p()
        rc = lib.barq_rocm_gguf_open(path.encode(), ctypes.byref(h))
        msg = lib.barq_rocm_last_error().decode()
        if rc == L.OK:
            lib.barq_rocm_gguf_close(h)
        return rc, msg

    W.write(p, KVS[:2], _tensors()[:2], magic=b"GGUX")
    assert open_rc(p)[0] == L.E_GGUF                        # Invalid magic (gguf.rs:257-262)
    W.write(p, KVS[:2], _tensors()[:2], version=4)
    rc, msg = open_rc(p)
    assert rc == L.E_GGUF and "Unsupported version" in msg   # version > 3 (gguf.rs:266-271)
    W.write(p, KVS[:2], _tensors()[:2], version=2)
    assert open_rc(p)[0] == L.OK
    W.write(p, [], [("t", [32], 4, bytes(20))])
    rc, msg = open_rc(p)
    assert rc == L.E_GGUF and "Unknown GGUF tensor type" in msg   # Q4_2 (id 4) is not in GgufTensorType
    # an unknown value type (13)
    import struct
    blob = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    open(p, "wb").write(blob)
    rc, msg = open_rc(p)
    assert rc == L.E_GGUF and "Unknown type: 13" in msg
    # a key that is not UTF-8 (String::from_utf8)
    blob = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xff\xfe" + struct.pack("<IB", 0, 1)
    open(p, "wb").write(blob)
    assert open_rc(p)[0] == L.E_GGUF
    # the header ends early: Error::Io
    W.write(p, KVS, _tensors())
    full = open(p, "rb").read()
    open(p, "wb").write(full[:40])
    assert open_rc(p)[0] == L.E_IO
    assert open_rc(str(tmp_path / "missing.gguf"))[0] == L.E_IO
    # the last tensor's data runs past the end: open succeeds, the read fails (read_exact)
    W.write(p, KVS[:1], _tensors()[:3], truncate=5)
    with GgufFile(p) as g:
        g.tensor(0)
        with pytest.raises(L.BarqError) as e:
            g.tensor(2)
        assert e.value.code == L.E_IO
        with pytest.raises(L.BarqError) as e:
            g.find("nope")
        assert e.value.code == L.E_INVALID and "Tensor not found" in str(e.value)


def test_alignment_key(tmp_path):
    p = str(tmp_path / "a.gguf")
    ts = _tensors()[:4]
    # general.alignment as a u32 sets the alignment (gguf.rs:279-282) ...
    d, offs = W.write(p, [("general.alignment", W.U32, 64)], ts, alignment=64)
    with GgufFile(p) as g:
        assert g.info()["alignment"] == 64 and g.info()["data_offset"] == d and d % 64 == 0
        for i, (_, _, _, raw) in enumerate(ts):
            assert g.tensor(i)["data"].tobytes() == raw
    # ... stored as any other type it is ignored and 32 is used
    d, _ = W.write(p, [("general.alignment", W.U64, 64)], ts, alignment=32)
    with GgufFile(p) as g:
        assert g.info()["alignment"] == 32 and g.info()["data_offset"] == d


def test_duplicate_tensor_names_resolve_to_the_first(tmp_path):
    p = str(tmp_path / "d.gguf")
    a = np.arange(8, dtype=np.float32).tobytes()
    b = np.ones(8, dtype=np.float32).tobytes()
    W.write(p, [], [("w", [8], 0, a), ("w", [8], 0, b)])
    with GgufFile(p) as g:
        assert g.find("w") == 0   # get_tensor_info: iter().find
