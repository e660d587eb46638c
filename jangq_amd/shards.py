"""Dtype-aligned safetensors shards: rewrite, verify, and read as zero-copy views.

A safetensors file is an 8-byte little-endian header length, a JSON header mapping each tensor
name to {dtype, shape, data_offsets: [begin, end)} relative to the data section, and the data
section. The format allows payloads in any order, so a mixed BF16/F16/U32 shard can place
uint32 code payloads at absolute offsets that are 2 mod 4; such a payload cannot be viewed
in place as a typed array and must be copied before it is uploaded.

The rewrite (jang-tools/jang_tools/format/aligned_safetensors.py:1-14, 85-180) changes the
container only: payloads are laid out by decreasing element size (ties by name), the JSON
header is padded with spaces so the data section starts at a multiple of max(8, largest
element size), and then every absolute payload offset is a multiple of its element size.
Names, dtypes, shapes, bytes and ``__metadata__`` are unchanged. The copy streams through a
bounded buffer, writes a temporary file beside the destination and installs it with an atomic
rename only once it is complete.

:func:`open_views` maps an aligned shard and returns each tensor as a view of the mapping
(no copy on the host); the bundle loader takes that route for shards that verify as aligned.
"""
from __future__ import annotations

import json
import mmap
import os
import shutil
import struct
from pathlib import Path

import numpy as np
import torch

# element size in bytes of each safetensors dtype (aligned_safetensors.py:26-46)
DTYPE_BYTES = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E5M2": 1, "F8_E4M3": 1, "F8_E4M3FN": 1, "F8_E8M0": 1,
    "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
    "I32": 4, "U32": 4, "F32": 4,
    "C64": 8, "I64": 8, "U64": 8, "F64": 8,
    "C128": 16,
}

# torch dtype of each safetensors dtype that a view can take directly
_TORCH = {
    "BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "I16": torch.int16,
    "U16": torch.uint16, "F16": torch.float16, "BF16": torch.bfloat16, "I32": torch.int32,
    "U32": torch.uint32, "F32": torch.float32, "I64": torch.int64, "U64": torch.uint64,
    "F64": torch.float64, "F8_E5M2": torch.float8_e5m2, "F8_E4M3FN": torch.float8_e4m3fn,
    "F8_E4M3": torch.float8_e4m3fn, "C64": torch.complex64, "C128": torch.complex128,
}

_MAX_HEADER = 100_000_000


def read_header(path) -> tuple[int, dict]:
    """(absolute start of the data section, header dict) of a safetensors file; ValueError for
    a truncated file, an implausible header length or a header that is not a JSON object."""
    path = Path(path)
    with path.open("rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: truncated safetensors length")
        n = struct.unpack("<Q", raw)[0]
        if not 0 < n < _MAX_HEADER:
            raise ValueError(f"{path}: invalid safetensors header length {n}")
        body = f.read(n)
        if len(body) != n:
            raise ValueError(f"{path}: truncated safetensors header")
    header = json.loads(body)
    if not isinstance(header, dict):
        raise ValueError(f"{path}: safetensors header is not an object")
    return 8 + n, header


def _entries(path, data_start: int, header: dict) -> list:
    """[(name, descriptor, begin, end, element size)] of every tensor, checked against the
    file's size."""
    size = Path(path).stat().st_size
    out = []
    for name, d in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(d, dict):
            raise ValueError(f"{path}: invalid descriptor for {name}")
        dt = d.get("dtype")
        if dt not in DTYPE_BYTES:
            raise ValueError(f"{path}: unsupported safetensors dtype {dt!r} for {name}")
        off = d.get("data_offsets")
        if not isinstance(off, list) or len(off) != 2:
            raise ValueError(f"{path}: invalid data_offsets for {name}")
        b, e = int(off[0]), int(off[1])
        if b < 0 or e < b:
            raise ValueError(f"{path}: invalid payload range for {name}")
        if data_start + e > size:
            raise ValueError(f"{path}: payload for {name} exceeds the file size")
        out.append((name, d, b, e, DTYPE_BYTES[dt]))
    return out


def aligned_layout(header: dict, entries: list) -> tuple[bytes, list]:
    """The rewritten header bytes (space-padded) and the payload order [(begin, end)] of the
    source: largest element size first, then by name, packed back to back from offset 0."""
    order = sorted(entries, key=lambda t: (-t[4], t[0]))
    new_header, cursor = {}, 0
    for name, d, b, e, _ in order:
        nd = dict(d)
        nd["data_offsets"] = [cursor, cursor + (e - b)]
        new_header[name] = nd
        cursor += e - b
    if "__metadata__" in header:
        new_header["__metadata__"] = header["__metadata__"]
    enc = json.dumps(new_header, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
    align = max([8] + [t[4] for t in entries])
    enc += b" " * ((-(8 + len(enc))) % align)
    return enc, [(b, e) for _, _, b, e, _ in order]


def rewrite_aligned(source, destination=None, *, chunk_bytes: int = 16 << 20) -> Path:
    """Stream ``source`` into a dtype-aligned container at ``destination`` (default: in place).
    The output is written to a temporary file beside the destination and renamed over it only
    when complete; on any error the temporary file is removed and the destination is as it
    was. Returns the destination path."""
    src = Path(source)
    dst = Path(destination) if destination is not None else src
    if chunk_bytes <= 0:
        raise ValueError("chunk_bytes must be positive")
    data_start, header = read_header(src)
    enc, spans = aligned_layout(header, _entries(src, data_start, header))
    dst.parent.mkdir(parents=True, exist_ok=True)
    tmp = dst.with_name(f".{dst.name}.aligned-{os.getpid()}.tmp")
    buf = bytearray(chunk_bytes)
    view = memoryview(buf)
    try:
        with src.open("rb") as fi, tmp.open("wb") as fo:
            fo.write(struct.pack("<Q", len(enc)))
            fo.write(enc)
            for b, e in spans:
                fi.seek(data_start + b)
                left = e - b
                while left:
                    got = fi.readinto(view[:min(left, chunk_bytes)])
                    if not got:
                        raise ValueError(f"{src}: payload truncated")
                    fo.write(view[:got])
                    left -= got
            fo.flush()
            os.fsync(fo.fileno())
        shutil.copymode(src, tmp)
        os.replace(tmp, dst)
    except BaseException:
        tmp.unlink(missing_ok=True)
        raise
    return dst


def verify_alignment(path) -> tuple[int, int]:
    """(tensor count, payloads whose absolute offset is not a multiple of their element
    size) of a safetensors file (aligned_safetensors.py:183-198)."""
    data_start, header = read_header(path)
    count = bad = 0
    for name, d in header.items():
        if name == "__metadata__":
            continue
        count += 1
        if (data_start + int(d["data_offsets"][0])) % DTYPE_BYTES[d["dtype"]]:
            bad += 1
    return count, bad


def repack_bundle(source_dir, output_dir) -> list:
    """Write an aligned copy of a bundle directory: every ``*.safetensors`` file rewritten,
    every other top-level file copied; the source is not modified (aligned_safetensors.py:
    201-217). Returns the rewritten shard names."""
    src, out = Path(source_dir), Path(output_dir)
    if src.resolve() == out.resolve():
        raise ValueError("bundle output must differ from source")
    out.mkdir(parents=True, exist_ok=True)
    done = []
    for p in sorted(src.iterdir()):
        if p.is_dir():
            continue
        if p.suffix == ".safetensors":
            rewrite_aligned(p, out / p.name)
            done.append(p.name)
        else:
            shutil.copy2(p, out / p.name)
    return done


class ShardViews:
    """A read-only mapping of an aligned shard; ``[name]`` is a torch tensor viewing the
    mapped bytes (no host copy; writes to it are refused by the mapping). The mapping stays
    open while any view of it lives."""

    def __init__(self, path):
        self.path = Path(path)
        self.data_start, header = read_header(self.path)
        self.entries = {t[0]: t for t in _entries(self.path, self.data_start, header)}
        self.metadata = header.get("__metadata__")
        for name, (_, d, b, _, es) in self.entries.items():
            if (self.data_start + b) % es:
                raise ValueError(f"{self.path}: {name} is not aligned to its {es}-byte "
                                 "elements (rewrite the shard with rewrite_aligned)")
            if d["dtype"] not in _TORCH:
                raise ValueError(f"{self.path}: no torch view for dtype {d['dtype']}")
        with self.path.open("rb") as f:
            size = os.fstat(f.fileno()).st_size
            self._map = mmap.mmap(f.fileno(), size, access=mmap.ACCESS_READ) if size else None
        self._bytes = (np.frombuffer(self._map, dtype=np.uint8) if self._map is not None
                       else np.zeros(0, np.uint8))

    def keys(self):
        return self.entries.keys()

    def __getitem__(self, name: str) -> torch.Tensor:
        _, d, b, e, _ = self.entries[name]
        raw = self._bytes[self.data_start + b:self.data_start + e]
        import warnings
        with warnings.catch_warnings():  # the mapping is read-only; torch warns about that
            warnings.simplefilter("ignore", UserWarning)
            t = torch.from_numpy(raw)
        return t.view(_TORCH[d["dtype"]]).reshape(d["shape"])


def open_views(path) -> ShardViews:
    """Views of every tensor of an aligned shard (ValueError when a payload is unaligned)."""
    return ShardViews(path)
