"""The build's GGUF reader (pbx_gguf_*) on the CPU, against files written by
tests/gguf_writer.py from the format the reference parses (gguf.js:76-194,
206-213, 429-450; streaming-loader.js:35-87).  No GPU is used: the reader
maps and parses the file on the host."""
import numpy as np
import pytest

import purebee_amd as pb
from purebee_amd.native import GGUF, PbxError
from tests import gguf_writer as gw

ALL_VALUES = [
    ("v.u8", gw.U8, 250), ("v.i8", gw.I8, -7), ("v.u16", gw.U16, 65000), ("v.i16", gw.I16, -30000),
    ("v.u32", gw.U32, 4000000000), ("v.i32", gw.I32, -2000000000), ("v.f32", gw.F32, 0.15625),
    ("v.bool", gw.BOOL, True), ("v.str", gw.STR, "héllo"), ("v.u64", gw.U64, 2 ** 40 + 3),
    ("v.i64", gw.I64, -(2 ** 40)), ("v.f64", gw.F64, -1e-300),
    ("v.arr_i32", gw.ARR, (gw.I32, [1, -2, 3])),
    ("v.arr_str", gw.ARR, (gw.STR, ["a", "", "ccc"])),
    ("v.arr_arr", gw.ARR, (gw.ARR, [(gw.U8, [1, 2]), (gw.STR, ["x"])])),
    ("v.empty", gw.STR, ""),
]


def small_tensors():
    rng = np.random.default_rng(1)
    return [
        ("a.f32", [5, 3], 0, rng.normal(0, 1, 15).astype(np.float32)),
        ("b.q4_0", [64, 2], 2, rng.integers(0, 256, 2 * 2 * 18, dtype=np.uint8)),
        ("c.f16", [7], 1, rng.normal(0, 1, 7).astype(np.float16)),
        ("d.q6_k", [256, 1], 14, rng.integers(0, 256, 210, dtype=np.uint8)),
        ("e.q8_0", [32, 1, 2], 8, rng.integers(0, 256, 2 * 34, dtype=np.uint8)),
    ]


@pytest.mark.parametrize("version", [2, 3])
@pytest.mark.parametrize("alignment", [32, 64, 1])
def test_reader_roundtrip(tmp_path, version, alignment):
    kv = list(ALL_VALUES)
    if alignment != 32:
        kv.append(("general.alignment", gw.U32, alignment))
    tensors = small_tensors()
    path = tmp_path / "t.gguf"
    offsets = gw.write(path, kv, tensors, version=version, alignment=alignment)
    with GGUF(path) as g:
        assert g.version == version and g.n_tensors == len(tensors) and g.n_kv == len(kv)
        assert g.get_int("v.u8") == 250 and g.get_int("v.i8") == -7
        assert g.get_int("v.u16") == 65000 and g.get_int("v.i16") == -30000
        assert g.get_int("v.u32") == 4000000000 and g.get_int("v.i32") == -2000000000
        assert g.get_float("v.f32") == 0.15625 and g.get_int("v.bool") == 1
        assert g.get_string("v.str") == "héllo" and g.get_string("v.empty") == ""
        assert g.get_int("v.u64") == 2 ** 40 + 3 and g.get_int("v.i64") == -(2 ** 40)
        assert g.get_float("v.f64") == -1e-300
        assert g.get_float("v.u32") == 4000000000.0   # integers read as floats too
        assert g.get_array("v.arr_i32") == (gw.I32, 3)
        assert g.get_array("v.arr_str") == (gw.STR, 3)
        assert g.get_array("v.arr_arr") == (gw.ARR, 2)
        with pytest.raises(PbxError):
            g.get_int("v.str")          # wrong value type
        with pytest.raises(PbxError):
            g.get_string("no.such.key")
        sizes = {0: 4, 1: 2}
        for i, (name, dims, t, data) in enumerate(tensors):
            info = g.tensor(i)
            assert info["name"] == name and info["type"] == t and info["dims"] == dims
            assert info["offset"] == offsets[i]
            n = int(np.prod(dims))
            # tensorByteSize, gguf.js:206-213
            want = n * sizes[t] if t in sizes else -(-n // (256 if t == 14 else 32)) * \
                {2: 18, 8: 34, 14: 210}[t]
            assert info["nbytes"] == want == np.asarray(data).nbytes
            assert np.array_equal(g.tensor_bytes(i), np.asarray(data).view(np.uint8).ravel())
            assert g.find(name) == i
        assert g.find("missing") == -1
        assert g.data_start % alignment == 0


def test_reader_rejects_bad_headers(tmp_path):
    blob, _ = gw.build([("k", gw.U32, 1)], small_tensors())
    cases = {
        "magic": b"GGUX" + blob[4:],
        "version1": gw.build([], [], header_version=1)[0],
        "version4": gw.build([], [], header_version=4)[0],
        "short": blob[:20],
    }
    for what, data in cases.items():
        p = tmp_path / f"{what}.gguf"
        p.write_bytes(data)
        with pytest.raises(PbxError) as e:
            GGUF(p)
        assert e.value.code in (-1, -5), what
    with pytest.raises(PbxError) as e:
        GGUF(tmp_path / "does_not_exist.gguf")
    assert e.value.code == -7


def test_reader_rejects_every_truncation(tmp_path):
    """Any prefix of a valid file is an error (or, past the tensor table, a
    tensor whose data runs off the end) -- never a read outside the file."""
    kv = list(ALL_VALUES)
    blob, offsets = gw.build(kv, small_tensors())
    last_end = offsets[-1] + 2 * 34
    p = tmp_path / "cut.gguf"
    for cut in list(range(0, 400)) + list(range(400, len(blob), 7)):
        p.write_bytes(blob[:cut])
        if cut >= last_end:
            GGUF(p).close()
            continue
        with pytest.raises(PbxError):
            GGUF(p)


def test_reader_rejects_unsized_types_and_bad_dims(tmp_path):
    # Q5_0 (6) is not in the reference's size table (gguf.js:36-49)
    p = tmp_path / "q5.gguf"
    gw.write(p, [], [("w", [32, 1], 6, np.zeros(22, np.uint8))])
    with pytest.raises(PbxError, match="unsupported tensor type 6"):
        GGUF(p)
    p2 = tmp_path / "dims.gguf"
    gw.write(p2, [], [("w", [0, 4], 0, np.zeros(0, np.float32))])
    with pytest.raises(PbxError, match="dimension"):
        GGUF(p2)
    p3 = tmp_path / "fivedims.gguf"
    gw.write(p3, [], [("w", [1, 1, 1, 1, 1], 0, np.zeros(1, np.float32))])
    with pytest.raises(PbxError, match="dimension count"):
        GGUF(p3)


def test_model_config_extraction(tmp_path):
    """extractConfig (gguf.js:429-450): architecture-prefixed keys, the
    reference's defaults, vocabulary from the tokenizer's token list."""
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, rope_theta=500000.0,
               rms_eps=1e-6, context_length=131072)
    emb = ("token_embd.weight", [256, 1000], 2, np.zeros(1000 * 8 * 18, np.uint8))
    q = ("blk.0.attn_q.weight", [256, 256], 8, np.zeros(256 * 8 * 34, np.uint8))
    out = ("output.weight", [256, 1000], 14, np.zeros(1000 * 210, np.uint8))
    p = tmp_path / "m.gguf"
    gw.write(p, gw.llama_kv(cfg, n_tokens=998), [emb, q, out])
    with GGUF(p) as g:
        c = g.model_config()
        assert (c["dim"], c["hidden_dim"], c["n_layers"], c["n_heads"], c["n_kv_heads"]) == \
            (256, 512, 2, 4, 2)
        assert c["head_dim"] == 64 and c["vocab_size"] == 998     # tokenizer count
        assert c["max_seq"] == 8192                                 # min(context, 8192)
        assert g.model_config(max_seq=300)["max_seq"] == 300
        assert (c["weight_type"], c["embed_type"], c["output_type"]) == (8, 2, 14)
        assert abs(c["rms_eps"] - 1e-6) < 1e-12 and c["rope_theta"] == 500000.0
    # defaults: head_count_kv = head_count, eps 1e-5, theta 10000, context 2048,
    # vocab = token_embd rows, tied head
    kv = [("general.architecture", gw.STR, "llama"), ("llama.embedding_length", gw.U32, 256),
          ("llama.feed_forward_length", gw.U32, 512), ("llama.block_count", gw.U32, 2),
          ("llama.attention.head_count", gw.U32, 8)]
    p2 = tmp_path / "d.gguf"
    gw.write(p2, kv, [emb, q])
    with GGUF(p2) as g:
        c = g.model_config()
        assert c["n_kv_heads"] == 8 and c["vocab_size"] == 1000 and c["output_type"] == -1
        assert c["max_seq"] == 2048 and c["rope_theta"] == 10000.0
        assert abs(c["rms_eps"] - 1e-5) < 1e-12
    # missing required keys
    p3 = tmp_path / "bad.gguf"
    gw.write(p3, kv[:2], [emb, q])
    with GGUF(p3) as g, pytest.raises(PbxError, match="block_count"):
        g.model_config()


def test_synth_writer_roundtrip(tmp_path):
    """purebee_amd.synth.write_gguf (the workloads' file writer) produces a
    file the reader parses into the same config and tensor bytes."""
    from purebee_amd import synth
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300,
               max_seq=64, weight_type=pb.TYPE_Q4_1, embed_type=pb.TYPE_Q6_K, output_type=pb.TYPE_F16,
               rope_theta=500000.0)
    p = tmp_path / "s.gguf"
    size = synth.write_gguf(p, cfg, seed=9)
    assert size == p.stat().st_size
    with GGUF(p) as g:
        c = g.model_config()
        assert (c["dim"], c["hidden_dim"], c["n_layers"], c["vocab_size"], c["max_seq"]) == \
            (256, 512, 2, 300, 64)
        assert (c["weight_type"], c["embed_type"], c["output_type"]) == \
            (pb.TYPE_Q4_1, pb.TYPE_Q6_K, pb.TYPE_F16)
        assert c["rope_theta"] == 500000.0
        for i, spec in enumerate(synth.tensor_specs(cfg)):
            name = synth.GGUF_NAMES[spec[0]] if spec[1] < 0 else \
                f"blk.{spec[1]}.{synth.GGUF_NAMES[spec[0]]}"
            j = g.find(name)
            assert j >= 0, name
            want = np.ascontiguousarray(synth.make_tensor(spec, 9, i)).view(np.uint8).ravel()
            assert np.array_equal(g.tensor_bytes(j), want), name
