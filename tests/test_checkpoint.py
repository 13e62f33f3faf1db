"""CPU tests of the safetensors reader and the GPT-OSS layer view
(physllm_amd/host/safetensors.hpp, gpt_oss_checkpoint.hpp) through tests/cpp/checkpoint_tool.

Files come from the `safetensors` package (an independent writer) or are written
byte by byte here for the malformed cases. The tool's view of every tensor (dtype,
shape, offset, size, FNV-1a of its bytes) must equal what the header JSON and the
data say when read by Python.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from physllm_amd import synthetic as syn
from tests import gpt_oss_ckpt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "tests", "cpp", "checkpoint_tool")


@pytest.fixture(scope="module")
def tool():
    if not os.path.exists(TOOL):
        from physllm_amd import build as b
        b.build_checkpoint_tools(verbose=False)
    return TOOL


def run(tool, *args):
    r = subprocess.run([tool, *map(str, args)], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout


def fnv1a(b: bytes) -> int:
    h = 1469598103934665603
    for c in b:
        h = ((h ^ c) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def python_view(path):
    """(name -> (dtype, shape, begin, nbytes, fnv)) from the file, read by Python."""
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    data = raw[8 + n:]
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        b, e = v["data_offsets"]
        out[k] = (v["dtype"], v["shape"], b, e - b, fnv1a(data[b:e]))
    return out, hdr.get("__metadata__", {})


def parse_dump(stdout):
    tens, meta = {}, {}
    for line in stdout.splitlines():
        f = line.split(" ")
        if f[0] == "tensor":
            shape = [int(x) for x in f[3][1:-1].split(",") if x]
            tens[f[1]] = (f[2], shape, int(f[4]), int(f[5]), int(f[6], 16))
        elif f[0] == "meta":
            meta[f[1]] = " ".join(f[2:])
    return tens, meta


def test_dump_matches_the_file(tool, tmp_path):
    t = {
        "a.u8": torch.arange(37, dtype=torch.uint8),
        "b.bf16": torch.randn(3, 5).to(torch.bfloat16),
        "c.f32": torch.randn(2, 3, 4),
        "d.i64": torch.arange(6, dtype=torch.int64).reshape(2, 3),
        "e.f16": torch.randn(7).to(torch.float16),
        "f.empty": torch.zeros(0, 4),
        "g.scalar": torch.tensor(3.5),
        "h.i32": torch.arange(10, dtype=torch.int32),
    }
    p = str(tmp_path / "one.safetensors")
    save_file(t, p, metadata={"format": "pt", "note": "two words"})
    rc, out = run(tool, "dump", p)
    assert rc == 0, out
    got, meta = parse_dump(out)
    exp, emeta = python_view(p)
    assert got == exp
    assert meta == emeta
    assert got["c.f32"][0] == "F32" and got["c.f32"][1] == [2, 3, 4] and got["g.scalar"][1] == []


def test_directory_of_shards_and_duplicates(tool, tmp_path):
    d = tmp_path / "ck"
    d.mkdir()
    save_file({"x": torch.ones(4), "y": torch.zeros(2, 2)}, str(d / "model-00001-of-00002.safetensors"))
    save_file({"z": torch.arange(3, dtype=torch.uint8)}, str(d / "model-00002-of-00002.safetensors"))
    (d / "notes.txt").write_text("not a shard")
    rc, out = run(tool, "dump", d)
    assert rc == 0, out
    assert out.splitlines()[0] == "shards 2"
    got, _ = parse_dump(out)
    assert sorted(got) == ["x", "y", "z"]
    save_file({"x": torch.ones(1)}, str(d / "model-00003-of-00003.safetensors"))
    rc, out = run(tool, "dump", d)
    assert rc == 3 and "more than one shard" in out
    empty = tmp_path / "empty"
    empty.mkdir()
    rc, out = run(tool, "dump", empty)
    assert rc == 3 and "no .safetensors" in out


def _write_raw(path, header: bytes, data: bytes, n_override=None):
    n = len(header) if n_override is None else n_override
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n) + header + data)


@pytest.mark.parametrize("case,header,data,expect", [
    ("short", None, b"", "shorter than"),
    ("hdr_past_end", b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}', b"\x00", "exceeds the file"),
    ("bad_json", b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}', b"\x00", "JSON"),
    ("trailing", b'{} x', b"", "trailing"),
    ("not_object", b'[1,2]', b"", "not a JSON object"),
    ("unknown_dtype", b'{"a":{"dtype":"Q9","shape":[1],"data_offsets":[0,1]}}', b"\x00", "unknown dtype"),
    ("size_mismatch", b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', b"\x00" * 8, "bytes for 2"),
    ("past_end", b'{"a":{"dtype":"U8","shape":[9],"data_offsets":[0,9]}}', b"\x00" * 8, "past the end"),
    ("overlap", b'{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]},"b":{"dtype":"U8","shape":[4],'
                b'"data_offsets":[2,6]}}', b"\x00" * 8, "overlap"),
    ("neg_dim", b'{"a":{"dtype":"U8","shape":[-1],"data_offsets":[0,0]}}', b"", "bad dimension"),
    ("dup_key", b'{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},"a":{"dtype":"U8","shape":[1],'
                b'"data_offsets":[1,2]}}', b"\x00\x00", "duplicate"),
    ("meta_not_str", b'{"__metadata__":{"k":1}}', b"", "must be strings"),
    ("bad_escape", b'{"a\\q":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}', b"\x00", "bad escape"),
])
def test_malformed_files_are_refused(tool, tmp_path, case, header, data, expect):
    p = str(tmp_path / f"{case}.safetensors")
    if header is None:
        open(p, "wb").write(b"\x01\x02\x03")
    elif case == "hdr_past_end":
        _write_raw(p, header, data, n_override=len(header) + 100)
    else:
        _write_raw(p, header, data)
    rc, out = run(tool, "dump", p)
    assert rc == 3, out
    assert expect in out, out


def test_json_string_escapes_in_names(tool, tmp_path):
    hdr = ('{"w\\"q\\\\\\/\\u00e9\\ud83d\\ude00":{"dtype":"U8","shape":[2],"data_offsets":[0,2]},'
           '"__metadata__":{"k":"v\\n"}}').encode()
    p = str(tmp_path / "esc.safetensors")
    _write_raw(p, hdr, b"\x07\x09")
    rc, out = run(tool, "dump", p)
    assert rc == 0, out
    got, _ = parse_dump(out)
    assert list(got) == ['w"q\\/é\U0001F600']
    assert got['w"q\\/é\U0001F600'][4] == fnv1a(b"\x07\x09")


def _layer_lines(out):
    return dict(line.split(" ", 1) for line in out.splitlines())


@pytest.mark.parametrize("naming,blocks_4d,f32", [("hf", True, False), ("orig", False, True), ("hf", False, False)])
def test_layer_view_both_namings(tool, tmp_path, naming, blocks_4d, f32):
    layers = [syn.make_layer(4, 64, 96, 2, seed=s) for s in (1, 2)]
    norms = [syn.make_x(1, 64, seed=s)[0] for s in (3, 4)]
    d = gpt_oss_ckpt.write_checkpoint(str(tmp_path / "ck"), layers, norms, top_k=2, naming=naming,
                                      blocks_4d=blocks_4d, f32_router=f32, eps=1e-6)
    for i in (0, 1):
        rc, out = run(tool, "layer", d, i)
        assert rc == 0, out
        v = _layer_lines(out)
        assert v["naming"] == ("huggingface" if naming == "hf" else "original")
        assert v["shape"] == "64 96 4"
        assert v["router_w"].endswith("F32" if f32 else "BF16")
        assert v["norm"] != "-" and v["gu_bias"] != "-"
        cfg = v["config"].split()
        assert cfg[:5] == ["64", "96", "4", "2", "2"] and cfg[7] == "1"
        if naming == "hf":
            assert float(cfg[5]) == pytest.approx(1e-6)
    rc, out = run(tool, "layer", d, 2)
    assert rc == 3 and "neither" in out


def test_layer_view_optional_and_wrong_tensors(tool, tmp_path):
    layer = syn.make_layer(4, 64, 96, 2, seed=1, with_bias=False)
    nw = syn.make_x(1, 64, seed=3)[0]
    d = gpt_oss_ckpt.write_checkpoint(str(tmp_path / "nobias"), [layer], [nw], top_k=2)
    rc, out = run(tool, "layer", d, 0)
    assert rc == 0, out
    v = _layer_lines(out)
    assert v["router_b"] == "-" and v["gu_bias"] == "-" and v["dn_bias"] == "-"
    # scales of the wrong shape are refused with the tensor's name
    good = syn.make_layer(4, 64, 96, 2, seed=1)
    bad = gpt_oss_ckpt.layer_tensors(good, 0, nw)
    bad["model.layers.0.mlp.experts.down_proj_scales"] = torch.zeros(4, 64, 2, dtype=torch.uint8)
    d2 = tmp_path / "bad"
    d2.mkdir()
    save_file(bad, str(d2 / "model.safetensors"))
    rc, out = run(tool, "layer", d2, 0)
    assert rc == 3 and "down_proj_scales" in out and "[4, 64, 3]" in out
    # blocks stored as another dtype are refused
    bad = gpt_oss_ckpt.layer_tensors(good, 0, nw)
    bad["model.layers.0.mlp.experts.gate_up_proj_blocks"] = torch.zeros(4, 192, 2, 16, dtype=torch.int16)
    d3 = tmp_path / "bad3"
    d3.mkdir()
    save_file(bad, str(d3 / "model.safetensors"))
    rc, out = run(tool, "layer", d3, 0)
    assert rc == 3 and "must be U8" in out


def test_mutated_headers_are_refused_or_read(tool, tmp_path):
    """Random corruptions of a valid file (header bytes, length field, truncation,
    inserted bytes) end in a clean read or a clean refusal, never a crash. (The same
    mutations ran 3000 times against an AddressSanitizer/UBSan build of the tool
    with no finding.)"""
    import random
    base = tmp_path / "base.safetensors"
    save_file({"a": torch.arange(37, dtype=torch.uint8), "b.x": torch.randn(3, 5).to(torch.bfloat16),
               "c": torch.randn(2, 3)}, str(base), metadata={"k": "v"})
    raw = base.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    rng = random.Random(7)
    p = tmp_path / "m.safetensors"
    for _ in range(200):
        b = bytearray(raw)
        kind = rng.randrange(4)
        if kind == 0:
            for _ in range(rng.randrange(1, 6)):
                b[8 + rng.randrange(n)] = rng.randrange(256)
        elif kind == 1:
            b = b[: rng.randrange(len(b))]
        elif kind == 2:
            b[0:8] = struct.pack("<Q", rng.choice([0, 1, n - 1, n + 1, 2**63, 2**64 - 1, rng.randrange(2**32)]))
        else:
            i = 8 + rng.randrange(n)
            b[i:i] = bytes(rng.randrange(256) for _ in range(rng.randrange(1, 4)))
        p.write_bytes(bytes(b))
        r = subprocess.run([tool, "dump", str(p)], capture_output=True, timeout=30)
        assert r.returncode in (0, 3), (kind, r.returncode, r.stderr[-300:])
