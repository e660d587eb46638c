"""Dtype-aligned safetensors shards (jang-tools/jang_tools/format/aligned_safetensors.py): the
rewrite keeps every name, dtype, shape, byte and the metadata (checked through the
safetensors library's own reader, an independent parser of the format), aligns every payload
to its element size, streams through small buffers, installs atomically and leaves the
destination alone on failure; the views of an aligned shard equal the tensors."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open

from jangq_amd import shards


def _raw_shard(path, items, metadata=None):
    """A safetensors file with payloads in exactly the given order (no reordering, no
    padding): items = [(name, dtype, shape, bytes)]."""
    header, cursor, blobs = {}, 0, []
    for name, dt, shape, data in items:
        header[name] = {"dtype": dt, "shape": list(shape),
                        "data_offsets": [cursor, cursor + len(data)]}
        cursor += len(data)
        blobs.append(data)
    if metadata is not None:
        header["__metadata__"] = metadata
    enc = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(enc)))
        f.write(enc)
        for b in blobs:
            f.write(b)
    return path


def _items(seed=0):
    rng = np.random.default_rng(seed)
    bf = rng.integers(0, 2**16, (3, 5), dtype=np.uint16)   # 30 bytes: shifts what follows by 2
    u32 = rng.integers(0, 2**32, (4, 7), dtype=np.uint64).astype(np.uint32)
    f32 = rng.standard_normal((6,)).astype(np.float32)
    u8 = rng.integers(0, 256, (5,), dtype=np.uint8)
    f64 = rng.standard_normal((2, 2))
    i16 = rng.integers(-2**15, 2**15, (3,), dtype=np.int16)
    return [("a.scales", "BF16", bf.shape, bf.tobytes()),
            ("b.weight", "U32", u32.shape, u32.tobytes()),
            ("c.bias", "F32", f32.shape, f32.tobytes()),
            ("d.mx", "U8", u8.shape, u8.tobytes()),
            ("e.f64", "F64", f64.shape, f64.tobytes()),
            ("f.i16", "I16", i16.shape, i16.tobytes()),
            ("g.empty", "U32", (0, 4), b"")]


def _tensors(path):
    with safe_open(str(path), framework="pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def test_rewrite_aligns_and_keeps_everything(tmp_path):
    src = _raw_shard(tmp_path / "s.safetensors", _items(), metadata={"format": "mlx", "k": "v"})
    n, bad = shards.verify_alignment(src)
    assert n == 7 and bad >= 2  # the U32 and F32 payloads after 30 bytes of BF16, at least
    before = src.read_bytes()
    dst = shards.rewrite_aligned(src, tmp_path / "out" / "d.safetensors", chunk_bytes=7)
    assert src.read_bytes() == before
    assert shards.verify_alignment(dst) == (7, 0)
    ta, ma = _tensors(src)
    tb, mb = _tensors(dst)
    assert ma == mb == {"format": "mlx", "k": "v"} and ta.keys() == tb.keys()
    for k in ta:
        assert ta[k].dtype == tb[k].dtype and ta[k].shape == tb[k].shape, k
        assert ta[k].view(torch.uint8).numpy().tobytes() == tb[k].view(torch.uint8).numpy().tobytes(), k
    data_start, header = shards.read_header(dst)
    assert data_start % 8 == 0
    order = sorted((v["data_offsets"][0], -shards.DTYPE_BYTES[v["dtype"]], k)
                   for k, v in header.items() if k != "__metadata__")  # (empty ones tie)
    sizes = [-es for _, es, _ in order]
    assert sizes == sorted(sizes, reverse=True)  # largest elements first
    # payloads packed back to back, the data section ending at the end of the file
    spans = sorted(tuple(v["data_offsets"]) for k, v in header.items() if k != "__metadata__")
    assert spans[0][0] == 0 and all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert data_start + spans[-1][1] == dst.stat().st_size
    # idempotent, and in place
    again = shards.rewrite_aligned(dst, tmp_path / "again.safetensors")
    assert again.read_bytes() == dst.read_bytes()
    shards.rewrite_aligned(src)
    assert src.read_bytes() == dst.read_bytes()
    assert not list(tmp_path.rglob(".*.tmp"))


def test_views_of_an_aligned_shard(tmp_path):
    src = _raw_shard(tmp_path / "s.safetensors", _items(1))
    with pytest.raises(ValueError, match="not aligned"):
        shards.open_views(src)
    dst = shards.rewrite_aligned(src, tmp_path / "d.safetensors")
    v = shards.open_views(dst)
    ref, _ = _tensors(dst)
    assert set(v.keys()) == set(ref)
    for k in ref:
        got = v[k]
        assert got.dtype == ref[k].dtype and got.shape == ref[k].shape, k
        assert torch.equal(got.view(torch.uint8) if got.numel() else got,
                           ref[k].view(torch.uint8) if got.numel() else ref[k]), k


def test_rewrite_failures_leave_the_destination(tmp_path):
    items = _items(2)
    src = _raw_shard(tmp_path / "s.safetensors", items)
    dst = tmp_path / "d.safetensors"
    dst.write_bytes(b"previous")
    trunc = tmp_path / "t.safetensors"
    trunc.write_bytes(src.read_bytes()[:-3])
    with pytest.raises(ValueError, match="exceeds the file size"):
        shards.rewrite_aligned(trunc, dst)
    assert dst.read_bytes() == b"previous" and not list(tmp_path.glob(".*.tmp"))
    bad = _raw_shard(tmp_path / "b.safetensors", [("x", "Q4", (2,), b"\0\0")])
    with pytest.raises(ValueError, match="unsupported safetensors dtype"):
        shards.rewrite_aligned(bad, dst)
    (tmp_path / "short").write_bytes(b"\1\0")
    with pytest.raises(ValueError, match="truncated safetensors length"):
        shards.read_header(tmp_path / "short")
    (tmp_path / "huge").write_bytes(struct.pack("<Q", 10**9) + b"{}")
    with pytest.raises(ValueError, match="header length"):
        shards.read_header(tmp_path / "huge")
    (tmp_path / "list").write_bytes(struct.pack("<Q", 2) + b"[]")
    with pytest.raises(ValueError, match="not an object"):
        shards.read_header(tmp_path / "list")
    with pytest.raises(ValueError, match="chunk_bytes"):
        shards.rewrite_aligned(src, dst, chunk_bytes=0)
    assert dst.read_bytes() == b"previous"


def test_repack_bundle(tmp_path):
    b = tmp_path / "bundle"
    b.mkdir()
    _raw_shard(b / "model-00001-of-00002.safetensors", _items(3))
    _raw_shard(b / "model-00002-of-00002.safetensors", _items(4)[::-1])
    (b / "config.json").write_text('{"a": 1}')
    (b / "sub").mkdir()
    src_bytes = {p.name: p.read_bytes() for p in b.iterdir() if p.is_file()}
    done = shards.repack_bundle(b, tmp_path / "out")
    assert done == ["model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
    out = tmp_path / "out"
    assert (out / "config.json").read_text() == '{"a": 1}' and not (out / "sub").exists()
    for name in done:
        assert shards.verify_alignment(out / name)[1] == 0
    assert {p.name: p.read_bytes() for p in b.iterdir() if p.is_file()} == src_bytes
    with pytest.raises(ValueError, match="differ"):
        shards.repack_bundle(b, b)


def test_loader_reads_aligned_shards_on_cpu_through_safetensors(tmp_path):
    """CPU loads copy (their tensors must not alias the read-only mapping)."""
    from jangq_amd import loader
    dst = shards.rewrite_aligned(_raw_shard(tmp_path / "s.safetensors", _items(5)),
                                 tmp_path / "d.safetensors")
    with loader._open_shard(dst, torch.device("cpu")) as f:
        assert not isinstance(f, loader._Views)
    with loader._open_shard(dst, torch.device("cuda")) as f:
        assert isinstance(f, loader._Views)  # no GPU call is made by opening
        t = f.get_tensor("b.weight")
        assert t.dtype == torch.uint32 and tuple(t.shape) == (4, 7)
