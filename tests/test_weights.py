"""The weight file (engine/src/weights.rs:38-74, layout tools/convert.py:117-150) on the host:
the writer's bytes against the documented layout packed by hand, the reader's records and
contents, and the checks that refuse malformed files and matrices (no GPU needed)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from violetto import _lib as L
from violetto.model import quantize_groups, quantize_rows
from violetto.weights import WeightFile, write_vlt


def _tensors():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(64, 512, generator=g) * 0.02
    q64, s64 = quantize_groups(w, 64)
    qr, sr = quantize_rows(w)
    return {
        "embed": (torch.randn(100, 512, generator=g) * 0.02).to(torch.bfloat16),
        "L00.scalars": torch.tensor([1.0, 0.9, 1.1, 1.0, 0.8, 1.2, 0.0, 0.0]),
        "L00.qkv": q64, "L00.qkv.scale": s64,
        "L00.o": qr, "L00.o.scale": sr,
        "L00.down": w.to(torch.bfloat16),
        "empty": torch.zeros(0, dtype=torch.float32),
    }


def test_layout_is_the_documented_one(tmp_path):
    """Header, first record and first tensor at the offsets the format documents."""
    path = tmp_path / "m.vlt"
    t = _tensors()
    write_vlt(path, t)
    b = path.read_bytes()
    magic, version, n, data_offset, r0, r1 = struct.unpack_from("<8sIIQII", b, 0)
    assert (magic, version, n, r0, r1) == (b"VIOLETTO", 1, len(t), 0, 0)
    assert data_offset == 16384 and len(b) % 16384 == 0
    name, dtype, ndim, s0, s1, s2, s3, off, nbytes = struct.unpack_from("<64sII4IQQ", b, 32)
    assert name.rstrip(b"\0") == b"embed" and dtype == 1 and ndim == 2 and (s0, s1, s2, s3) == (100, 512, 0, 0)
    assert off == 0 and nbytes == 100 * 512 * 2
    assert b[data_offset:data_offset + nbytes] == t["embed"].view(torch.uint8).numpy().tobytes()
    # the second tensor starts at the next 256-byte boundary
    off1 = struct.unpack_from("<Q", b, 32 + 128 + 88)[0]
    assert off1 == -(-nbytes // 256) * 256


def test_reader_records_and_contents(tmp_path):
    path = tmp_path / "m.vlt"
    t = _tensors()
    write_vlt(path, t)
    wf = WeightFile(path)
    assert len(wf) == len(t)
    names = [wf.info(i).name.decode() for i in range(len(wf))]
    assert names == list(t)
    for name, x in t.items():
        info = wf.find(name)
        assert tuple(info.shape[: info.ndim]) == tuple(x.shape)
        got = wf.read(name)
        want = x.view(torch.int16).numpy().view(np.uint16) if x.dtype == torch.bfloat16 else x.numpy()
        assert np.array_equal(got, want), name
    with pytest.raises(L.SvError, match="weight file has no tensor missing"):
        wf.find("missing")
    # matrices are checked before any device memory is needed
    with pytest.raises(L.SvError, match="expected I8 \\[64, 256\\], found I8 \\[64, 512\\]"):
        wf.matrix("L00.qkv", 64, 256)
    with pytest.raises(L.SvError, match="not uploaded"):
        wf.matrix("L00.qkv", 64, 512)
    wf.close()


def _write_raw(path, records, data=b"", n=None, version=1, magic=b"VIOLETTO"):
    head = struct.pack("<8sIIQII", magic, version, len(records) if n is None else n, 16384, 0, 0)
    body = head + b"".join(records)
    body += b"\0" * (16384 - len(body)) + data
    path.write_bytes(body)


def _rec(name, dtype, shape, off, nbytes):
    sh = list(shape) + [0] * (4 - len(shape))
    return struct.pack("<64sII4IQQ24x", name.encode(), dtype, len(shape), *sh, off, nbytes)


@pytest.mark.parametrize("case,msg", [
    ("magic", "not a version-1 violetto weight file"),
    ("version", "not a version-1 violetto weight file"),
    ("dtype", "x: unknown dtype 5"),
    ("bytes", "x: 12 bytes for a \\[4, 0, 0, 0\\] F32 shape"),
    ("past_end", "x: bytes past the end of the file"),
    ("twice", "x: two tensors of this name"),
    ("records", "records do not fit the file"),
    # dims whose product wraps in 64 bits to nbytes / 4 = 4 elements
    ("wrap_shape", "x: 16 bytes for a \\[4, 242243305, 49477, 384773\\] F32 shape"),
    # offset + nbytes wraps past zero
    ("wrap_offset", "x: bytes past the end of the file"),
    ("misaligned", "x: offset 16 is not a multiple of 256"),
    ("long_name", "record 0 has a 64-byte name with no NUL"),
])
def test_malformed_files_refused(tmp_path, case, msg):
    p = tmp_path / "bad.vlt"
    data = b"\0" * 256
    if case == "magic":
        _write_raw(p, [_rec("x", 0, [4], 0, 16)], data, magic=b"VIOLETTA")
    elif case == "version":
        _write_raw(p, [_rec("x", 0, [4], 0, 16)], data, version=2)
    elif case == "dtype":
        _write_raw(p, [_rec("x", 5, [4], 0, 16)], data)
    elif case == "bytes":
        _write_raw(p, [_rec("x", 0, [4], 0, 12)], data)
    elif case == "past_end":
        _write_raw(p, [_rec("x", 0, [4], 256, 16)], data)
    elif case == "twice":
        _write_raw(p, [_rec("x", 0, [4], 0, 16), _rec("x", 0, [4], 256, 16)], data * 2)
    elif case == "wrap_shape":
        # 4 (2^62 + 1) = 2^64 + 4: the product wraps to 4 elements, 16 bytes
        _write_raw(p, [_rec("x", 0, [4, 5 * 5581 * 8681, 49477, 384773], 0, 16)], data)
    elif case == "wrap_offset":
        _write_raw(p, [_rec("x", 0, [4], 2**64 - 256, 16)], data)
    elif case == "misaligned":
        _write_raw(p, [_rec("x", 0, [4], 16, 16)], data)
    elif case == "long_name":
        _write_raw(p, [_rec("y" * 64, 0, [4], 0, 16)], data)
    else:
        _write_raw(p, [_rec("x", 0, [4], 0, 16)], data, n=200)
    with pytest.raises(L.SvError, match=msg):
        WeightFile(p)


def test_matrix_groups_checked(tmp_path):
    """model.rs:94-99: int8 groups must be a power of two from 8 to 256 that divides k (one
    group per row, the configurations' format, also accepted); the scale must exist."""
    g = torch.Generator().manual_seed(1)
    w = torch.randn(16, 96, generator=g)
    q, _ = quantize_rows(w)
    path = tmp_path / "g.vlt"
    write_vlt(path, {"a": q, "a.scale": torch.ones(16, 5, dtype=torch.bfloat16),  # 96 / 5 is no group
                     "b": q, "b.scale": torch.ones(16, 24, dtype=torch.bfloat16),  # groups of 4
                     "c": q})
    wf = WeightFile(path)
    with pytest.raises(L.SvError, match="a.scale: 5 groups per row of 96"):
        wf.matrix("a", 16, 96)
    with pytest.raises(L.SvError, match="b.scale: 24 groups per row of 96"):
        wf.matrix("b", 16, 96)
    with pytest.raises(L.SvError, match="weight file has no tensor c.scale"):
        wf.matrix("c", 16, 96)


def test_limite_tensors_round_trip(tmp_path):
    """A Limite-layout model (extras and an int8 head of groups of 64) written under the
    reference's names (tools/convert.py:76-113) reads back with every name, dtype and shape
    model.rs:109-141 asks for, contents equal."""
    from violetto.model import ModelShape, SyntheticModel, generate_extras, rope_freq
    from violetto.weights import reference_tensors

    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=8)
    model = SyntheticModel.generate(shape, seed=2, group=64).with_extras(generate_extras(shape, seed=3, window=48))
    model = model.with_head(64)
    t = reference_tensors(model, rope_freq(500000.0, 64))
    path = tmp_path / "limite.vlt"
    write_vlt(path, t)
    wf = WeightFile(path)
    want = {"embed": (1, (512, 256)), "value_embed": (1, (512, 128)), "rope_freq": (0, (32,)),
            "mudd.dense1": (0, (32, 256)), "mudd.mix": (0, (2, 2, 3, 33)), "head": (2, (512, 256)),
            "head.scale": (1, (512, 4))}
    for i in range(8):
        want[f"L{i:02d}.attn_gate"] = (0, (4, 64))
        want[f"L{i:02d}.xsa"] = (0, (4,))
        want[f"L{i:02d}.qkv"] = (2, (512, 256))
        want[f"L{i:02d}.qkv.scale"] = (1, (512, 4))
        if i % 3 == 1:
            want[f"L{i:02d}.ve_gate"] = (0, (2, 12))
        else:
            assert not wf.has(f"L{i:02d}.ve_gate")
    for name, (dt, shp) in want.items():
        wf.check(name, dt, shp)
    np.testing.assert_array_equal(wf.read("L04.xsa"), model.extras.xsa[4].numpy())
    np.testing.assert_array_equal(wf.read("mudd.mix")[:2], model.extras.mudd_mix.numpy())
    np.testing.assert_array_equal(wf.read("head"), model.head[0].numpy())
    with pytest.raises(ValueError, match="expected dtype"):
        wf.check("L00.xsa", 1, (4,))
    wf.close()


def test_drafter_tensors_round_trip(tmp_path):
    """A drafter written under export.py's names (tools/spec/export.py:28-60) reads back with
    the names, dtypes and shapes drafter.rs:145-241 asks for: meta (layers, taps, block, window,
    vocabulary, the taps), the head in int8 groups of 8, corrections padded to 64-row tiles."""
    from violetto.drafter import SyntheticDrafter, drafter_tensors
    from violetto.model import ModelShape

    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=384, vocab=512, vocab_real=500,
                       n_layers=6)
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(2, 5), v=128, window=48, seed=1)
    path = tmp_path / "drafter.vlt"
    write_vlt(path, drafter_tensors(d))
    wf = WeightFile(path)
    np.testing.assert_array_equal(wf.read("meta"), np.array([2, 2, 8, 48, 128, 2, 5], np.float32))
    want = {"fc.0": (2, (256, 256)), "fc.1": (2, (256, 256)), "kv_all": (2, (512, 256)), "inject": (2, (256, 256)),
            "head": (2, (128, 256)), "head.scale": (1, (128, 32)), "mask_emb": (0, (256,)), "vocab": (0, (128,)),
            "D01.qkv": (2, (512, 256)), "D01.gate_up": (2, (768, 256)), "D01.down": (2, (256, 384)),
            "D00.conv3.base": (0, (2, 256)), "D00.conv3.corr": (2, (64, 256)), "D00.conv3.corr.scale": (1, (64, 4))}
    for name, (dt, shp) in want.items():
        wf.check(name, dt, shp)
    np.testing.assert_array_equal(wf.read("vocab").astype(np.int64), d.vocab.numpy())
    np.testing.assert_array_equal(wf.read("head"), d.mats["head"][0].numpy())
