"""The GGUF container (parse_gguf_file E:376-413): the library's parser
against the reference's own parser compiled in place (oracle/_ref) and the
writer's layout, on synthetic files; host only, no GPU."""
import os

import numpy as np
import pytest

import gguf_writer as gw
import qmm_hip
import synth
from oracle import TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0

LONG = "blk.0." + "x" * 200 + ".weight"


def _model_like():
    w_gate = synth.weights(TYPE_Q4_K, 32, 2560, seed=1).tobytes()
    w_down = synth.weights(TYPE_Q6_K, 16, 512, seed=2).tobytes()
    emb = synth.weights(TYPE_Q8_0, 10, 64, seed=3).tobytes()
    norm = np.linspace(0.5, 1.5, 2560, dtype=np.float32).tobytes()
    kv = [("general.architecture", gw.STR, "qwen3"),
          ("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["<a>", "b", "ccc"])),
          ("some.f32s", gw.ARR, (gw.F32, [1.0, 2.0, 3.5])),
          ("some.flag", gw.BOOL, True),
          ("some.u64", gw.U64, 123456789012),
          ("some.i16", gw.I16, -7)]
    ts = [("blk.0.ffn_gate.weight", [2560, 32], TYPE_Q4_K, w_gate),
          ("blk.0.ffn_down.weight", [512, 16], TYPE_Q6_K, w_down),
          ("output_norm.weight", [2560], 0, norm),
          ("token_embd.weight", [64, 10], TYPE_Q8_0, emb),
          (LONG, [256, 1, 1, 2], TYPE_Q4_K, synth.weights(TYPE_Q4_K, 2, 256, seed=4).tobytes())]
    return kv, ts


@pytest.mark.parametrize("version,align", [(3, None), (3, 64), (2, 32), (3, 256)])
def test_parse_matches_reference(tmp_path, ref, version, align):
    kv, ts = _model_like()
    path = tmp_path / "m.gguf"
    data, data_off, offs = gw.write(path, kv, ts, version=version, align=align)
    with qmm_hip.Gguf(str(path)) as g:
        h = g.header()
        mine = g.tensors()
        assert h["version"] == version and h["alignment"] == (align or 32)
        assert h["data_offset"] == data_off and h["n_tensors"] == len(ts)
        for t, (name, dims, ty, raw), o in zip(mine, ts, offs):
            assert t["name"] == name[:127] and t["type"] == ty and t["rel_offset"] == o
            assert t["abs_offset"] == data_off + o and t["dims"][:len(dims)] == dims
            assert bytes(g.data(t["name"]))[:len(raw)] == raw[:t["byte_size"]]
        assert g.find("blk.0.ffn_down.weight")["type"] == TYPE_Q6_K
        assert g.find("no.such.tensor") is None
    al, do, theirs = ref.gguf_parse(data)
    assert (al, do) == (h["alignment"], h["data_offset"])
    for a, b in zip(mine, theirs):
        assert a == b


def test_byte_sizes_follow_compute_ggml_bytes(tmp_path):
    kv, ts = _model_like()
    path = tmp_path / "m.gguf"
    gw.write(path, kv, ts)
    with qmm_hip.Gguf(str(path)) as g:
        sizes = [t["byte_size"] for t in g.tensors()]
    assert sizes == [32 * 1440, 16 * 420, 2560 * 4, 10 * 68, 2 * 144]


@pytest.mark.parametrize("mutate", ["magic", "v1", "v4", "ndims0", "ndims5", "truncated"])
def test_rejected_like_the_reference(tmp_path, ref, mutate):
    kv, ts = _model_like()
    if mutate == "ndims0":
        ts[0] = (ts[0][0], [], ts[0][2], ts[0][3])
    if mutate == "ndims5":
        ts[0] = (ts[0][0], [256, 1, 1, 1, 10], ts[0][2], ts[0][3])
    version = {"v1": 1, "v4": 4}.get(mutate, 3)
    data, _, _ = gw.gguf_bytes(kv, ts, version=version)
    if mutate == "magic":
        data = b"GGUG" + data[4:]
    if mutate == "truncated":
        data = data[:200]
    path = tmp_path / "bad.gguf"
    path.write_bytes(data)
    assert ref.gguf_parse(data) is None
    with pytest.raises(qmm_hip.QmmError):
        qmm_hip.Gguf(str(path))


def test_tensor_past_end_is_an_error(tmp_path, ref):
    """A difference from the reference (which accepts the table): tensor
    bytes outside the file are rejected with QMM_ESHAPE."""
    kv, ts = _model_like()
    data, _, _ = gw.gguf_bytes(kv, ts)
    data = data[:-100]
    path = tmp_path / "short.gguf"
    path.write_bytes(data)
    assert ref.gguf_parse(data) is not None
    with pytest.raises(qmm_hip.QmmError) as e:
        qmm_hip.Gguf(str(path))
    assert e.value.status == 3
