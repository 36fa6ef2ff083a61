"""EXL3 checkpoint ingestion on the host: the safetensors header inventory
and its validation, the packed matrices it holds, their H128-block shards,
loading a packed weight, and the expert pointer / metadata tables the MoE
kernels read.

Mirrors the reference's CPU side:
  * ``read_headers`` / ``Exl3Manifest`` / ``PackedMatrix`` /
    ``aligned_shard`` / ``block_shard``: vllm_sm80/kernels/exl3/utils.py:
    57-288 (header parse and extent checks, the per-matrix tensor set
    {trellis, suh, svh, mcg | mul1}, codebook multipliers, admissible rates,
    orphan and conflict checks);
  * ``Exl3PackedWeight``: quant.py:382-466 (H128-block slices, padded /
    logical geometry, ``load`` copying the trellis tile columns and the
    scale slices of each shard);
  * ``expert_tables``: quant.py:1105-1134 (packed_ptrs [E][3][3] = trellis,
    suh, svh device addresses; packed_meta [E][3][4] = padded_in,
    padded_out, bits_x2, codebook).
No byte of the checkpoint is interpreted beyond the safetensors header
(JSON) and the codebook marker scalars; payloads are read through
safetensors' own loader.
"""

from __future__ import annotations

import json
import math
import struct
from dataclasses import dataclass
from pathlib import Path

import torch

DTYPE_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "I16": 2, "F16": 2, "BF16": 2, "I32": 4, "F32": 4,
               "I64": 8, "F64": 8}
FP8_DTYPE_BYTES = {"F8_E4M3": 1, "F8_E5M2": 1, "F8_E8M0": 1}
# codebook marker tensor -> (codebook id, multiplier it must hold)
MARKERS = {"mcg": (1, 0xCBAC1FED), "mul1": (2, 0x83DCD12D)}
_HEADER_LIMIT = 100_000_000


def _no_duplicate_keys(pairs):
    out = {}
    for key, value in pairs:
        if key in out:
            raise ValueError(f"Duplicate JSON key: {key}")
        out[key] = value
    return out


@dataclass(frozen=True)
class TensorHeader:
    name: str
    path: Path
    dtype: str
    shape: tuple
    data_start: int
    data_offsets: tuple

    @property
    def offset(self) -> int:
        return self.data_start + self.data_offsets[0]

    @property
    def nbytes(self) -> int:
        return self.data_offsets[1] - self.data_offsets[0]

    def read_bytes(self) -> bytes:
        with self.path.open("rb") as f:
            f.seek(self.offset)
            data = f.read(self.nbytes)
        if len(data) != self.nbytes:
            raise ValueError(f"Truncated EXL3 tensor: {self.name}")
        return data


def _header(path: Path):
    size = path.stat().st_size
    with path.open("rb") as f:
        prefix = f.read(8)
        if len(prefix) != 8:
            raise ValueError(f"Truncated safetensors header: {path.name}")
        (length,) = struct.unpack("<Q", prefix)
        if length > min(size - 8, _HEADER_LIMIT):
            raise ValueError(f"Invalid safetensors header size: {path.name}")
        header = json.loads(f.read(length), object_pairs_hook=_no_duplicate_keys)
    return header, 8 + length, size


def read_metadata(path: Path) -> dict:
    meta = _header(Path(path))[0].get("__metadata__", {})
    if not isinstance(meta, dict):
        raise ValueError(f"Invalid safetensors metadata: {Path(path).name}")
    return meta


def read_headers(path, dtype_bytes=DTYPE_BYTES) -> dict:
    """name -> TensorHeader of one safetensors file, after checking that
    every extent matches its dtype and shape and that the extents tile the
    payload exactly (no gap, overlap or trailing bytes)."""
    path = Path(path)
    header, start, size = _header(path)
    tensors = {}
    for name, entry in header.items():
        if name == "__metadata__":
            continue
        dtype, shape, offsets = entry["dtype"], entry["shape"], entry["data_offsets"]
        if dtype not in dtype_bytes or any(type(d) is not int or d < 0 for d in shape):
            raise ValueError(f"Invalid dtype/shape: {name}")
        if (len(offsets) != 2 or any(type(v) is not int for v in offsets)
                or not 0 <= offsets[0] <= offsets[1] <= size - start
                or offsets[1] - offsets[0] != math.prod(shape) * dtype_bytes[dtype]):
            raise ValueError(f"Invalid tensor extent: {name}")
        tensors[name] = TensorHeader(name, path, dtype, tuple(shape), start, tuple(offsets))
    end = 0
    for t in sorted(tensors.values(), key=lambda t: t.data_offsets):
        if t.data_offsets[0] != end:
            raise ValueError(f"Overlapping or noncontiguous extent: {t.name}")
        end = t.data_offsets[1]
    if start + end != size:
        raise ValueError(f"Unaccounted safetensors payload: {path.name}")
    return tensors


@dataclass(frozen=True)
class PackedMatrix:
    prefix: str
    padded_in: int
    padded_out: int
    bits_x2: int
    codebook: int
    marker: str

    @property
    def keys(self) -> tuple:
        return tuple(f"{self.prefix}.{s}" for s in ("trellis", "suh", "svh", self.marker))

    def validate_logical(self, logical_in: int, logical_out: int) -> None:
        if (-(-logical_in // 128) * 128 != self.padded_in
                or -(-logical_out // 128) * 128 != self.padded_out):
            raise ValueError(f"EXL3 logical/padded geometry mismatch: {self.prefix}")


def admissible_rate(bits_x2: int, codebook: int) -> bool:
    """Even rates 1..8 bits for both codebooks, odd half-bit rates for mul1."""
    return bits_x2 in range(2, 17, 2) or (codebook == 2 and bits_x2 in (3, 5, 7))


class Exl3Manifest:
    """The checkpoint's tensors by name (every ``*.safetensors`` in the
    directory; with ``select_by_index`` only those the index's weight_map
    names, each from the file it names) and its packed matrices by prefix."""

    def __init__(self, directory, select_by_index: bool = False):
        self.directory = Path(directory)
        self.tensors: dict = {}
        self.matrices: dict = {}
        self.ple_tables: dict = {}
        self.unselected = 0
        paths = sorted(self.directory.glob("*.safetensors"))
        if not paths:
            raise ValueError("EXL3 requires local safetensors checkpoint files")
        index = self.directory / "model.safetensors.index.json"
        entries = None
        if index.exists():
            entries = json.loads(index.read_text(), object_pairs_hook=_no_duplicate_keys)["weight_map"]
        elif select_by_index:
            raise ValueError("A hybrid EXL3 checkpoint selects its tensors with "
                             "model.safetensors.index.json, which it lacks")
        dtype_bytes = DTYPE_BYTES | FP8_DTYPE_BYTES if select_by_index else DTYPE_BYTES
        for path in paths:
            for name, tensor in read_headers(path, dtype_bytes).items():
                if select_by_index and entries.get(name) != path.name:
                    self.unselected += 1
                    continue
                if name in self.tensors:
                    raise ValueError(f"Duplicate EXL3 source tensor: {name}")
                self.tensors[name] = tensor
        self.tensors = dict(sorted(self.tensors.items()))
        if entries is not None:
            for name, filename in entries.items():
                t = self.tensors.get(name)
                if t is None or t.path.name != filename:
                    raise ValueError(f"EXL3 index/header conflict: {name}")
        for name, tensor in self.tensors.items():
            if not name.endswith(".trellis"):
                continue
            prefix = name[: -len(".trellis")]
            if prefix.endswith(".ngram_embedding"):
                self.ple_tables[prefix] = tensor  # row-decoded tables (ple_decode_out)
                continue
            self.matrices[prefix] = self._matrix(prefix, tensor)
        packed = {k for m in self.matrices.values() for k in m.keys}
        for name in self.tensors:
            if name.endswith((".suh", ".svh", ".mcg", ".mul1")) and name not in packed:
                if not any(name.startswith(p + ".") for p in self.ple_tables):
                    raise ValueError(f"Orphan EXL3 quantization tensor: {name}")

    def expect(self, name: str, dtype: str, shape: tuple) -> TensorHeader:
        t = self.tensors.get(name)
        if t is None or t.dtype != dtype or t.shape != shape:
            raise ValueError(f"Missing or incompatible EXL3 tensor: {name}")
        return t

    def _matrix(self, prefix: str, trellis: TensorHeader) -> PackedMatrix:
        if trellis.dtype != "I16" or len(trellis.shape) != 3:
            raise ValueError(f"Invalid EXL3 trellis: {prefix}")
        tk, tn, words = trellis.shape
        k, n = tk * 16, tn * 16
        if k <= 0 or n <= 0 or k % 128 or n % 128 or words % 8:
            raise ValueError(f"Invalid EXL3 tile geometry: {prefix}")
        self.expect(f"{prefix}.suh", "F16", (k,))
        self.expect(f"{prefix}.svh", "F16", (n,))
        markers = [m for m in MARKERS if f"{prefix}.{m}" in self.tensors]
        if len(markers) != 1:
            raise ValueError(f"Missing/conflicting EXL3 codebook: {prefix}")
        marker = markers[0]
        codebook, value = MARKERS[marker]
        header = self.expect(f"{prefix}.{marker}", "I32", ())
        if struct.unpack("<I", header.read_bytes())[0] != value:
            raise ValueError(f"Unsupported EXL3 codebook multiplier: {prefix}")
        bits_x2 = words // 8
        if not admissible_rate(bits_x2, codebook):
            raise ValueError(f"Unsupported EXL3 bitrate/codebook: {prefix}")
        if f"{prefix}.weight" in self.tensors:
            raise ValueError(f"Conflicting dense and EXL3 weights: {prefix}")
        return PackedMatrix(prefix, k, n, bits_x2, codebook, marker)


def aligned_shard(logical: int, padded: int, rank: int, size: int) -> slice:
    """Rank ``rank`` of ``size`` equal shards of whole H128 blocks."""
    if size <= 0 or not 0 <= rank < size:
        raise ValueError("Invalid EXL3 shard rank/size")
    if size == 1:
        return slice(0, padded)
    if logical != padded or logical % size or (logical // size) % 128:
        raise ValueError(f"EXL3 TP cuts must preserve H128 blocks: {logical=} {padded=} {size=}")
    width = logical // size
    return slice(rank * width, (rank + 1) * width)


def block_shard(logical: int, padded: int, rank: int, size: int, rotation: int = 0) -> slice:
    """Whole H128 blocks split as evenly as they go: the first
    ``blocks % size`` chunks take one block more, and rank ``rank`` takes
    chunk ``(rank + rotation) % size``."""
    if size <= 0 or not 0 <= rank < size or rotation < 0:
        raise ValueError("Invalid EXL3 shard rank/size/rotation")
    if size == 1:
        return slice(0, padded)
    if logical != padded or logical % 128:
        raise ValueError(f"EXL3 TP cuts must preserve H128 blocks: {logical=} {padded=}")
    base, extra = divmod(logical // 128, size)
    if base == 0:
        raise ValueError(f"EXL3 cannot give {size} ranks a block of {logical}")
    chunk = (rank + rotation) % size
    start = chunk * base + min(chunk, extra)
    return slice(start * 128, (start + base + (chunk < extra)) * 128)


class Exl3PackedWeight:
    """One packed matrix (or a shard of whole H128 blocks of it): trellis
    int16 [padded_in / 16][padded_out / 16][8 bits_x2], suh / svh fp16."""

    def __init__(self, matrix: PackedMatrix, logical_in: int, logical_out: int,
                 input_slice: slice, output_slices: list):
        for part, limit in [(input_slice, matrix.padded_in)] + [(p, matrix.padded_out)
                                                                for p in output_slices]:
            if (part.step is not None or not 0 <= part.start < part.stop <= limit
                    or part.start % 128 or part.stop % 128):
                raise ValueError("EXL3 shards must select complete H128 blocks")
        self.matrix = matrix
        self.logical_in = logical_in
        self.logical_out = logical_out
        self.input_slice = input_slice
        self.output_slices = list(output_slices)
        self.padded_in = input_slice.stop - input_slice.start
        self.padded_out = sum(s.stop - s.start for s in output_slices)
        if not 0 < logical_in <= self.padded_in or not 0 < logical_out <= self.padded_out:
            raise ValueError("EXL3 logical dimensions exceed assigned packed blocks")
        self.trellis = torch.empty((self.padded_in // 16, self.padded_out // 16, 8 * matrix.bits_x2),
                                   dtype=torch.int16)
        self.suh = torch.empty(self.padded_in, dtype=torch.float16)
        self.svh = torch.empty(self.padded_out, dtype=torch.float16)
        self.loaded = False

    def load(self, manifest: Exl3Manifest) -> None:
        """Copies this shard's trellis tile columns and scale slices out of
        the checkpoint."""
        from safetensors import safe_open

        prefix = self.matrix.prefix
        ks = slice(self.input_slice.start // 16, self.input_slice.stop // 16)

        def open_slice(suffix):
            header = manifest.tensors[f"{prefix}.{suffix}"]
            handle = safe_open(str(header.path), framework="pt")
            return handle.get_slice(header.name)

        packed = open_slice("trellis")
        offset = 0
        for part in self.output_slices:
            ns = slice(part.start // 16, part.stop // 16)
            width = ns.stop - ns.start
            self.trellis[:, offset:offset + width].copy_(packed[ks, ns, :])
            offset += width
        for suffix, dest, parts in (("suh", self.suh, [self.input_slice]),
                                    ("svh", self.svh, self.output_slices)):
            data = open_slice(suffix)
            offset = 0
            for part in parts:
                width = part.stop - part.start
                dest[offset:offset + width].copy_(data[part])
                offset += width
        self.loaded = True

    def to(self, device) -> "Exl3PackedWeight":
        self.trellis = self.trellis.to(device)
        self.suh = self.suh.to(device)
        self.svh = self.svh.to(device)
        return self


def load_matrix(manifest: Exl3Manifest, prefix: str, logical_in: int, logical_out: int,
                device=None) -> Exl3PackedWeight:
    """The whole matrix ``prefix`` (one GPU: no shard), validated against its
    logical geometry and loaded."""
    matrix = manifest.matrices.get(prefix)
    if matrix is None:
        raise ValueError(f"No EXL3 matrix {prefix}")
    matrix.validate_logical(logical_in, logical_out)
    weight = Exl3PackedWeight(matrix, logical_in, logical_out, slice(0, matrix.padded_in),
                              [slice(0, matrix.padded_out)])
    weight.load(manifest)
    return weight.to(device) if device is not None else weight


def expert_tables(experts, device) -> tuple:
    """(packed_ptrs int64 [E][3][3], packed_meta int64 [E][3][4]) for the MoE
    kernels from loaded expert weights [E][gate, up, down] on the device."""
    ptrs, meta = [], []
    for expert in experts:
        if len(expert) != 3:
            raise ValueError("EXL3 expert assignment is incomplete or duplicated")
        p, m = [], []
        for w in expert:
            if not w.loaded or not all(t.is_cuda for t in (w.trellis, w.suh, w.svh)):
                raise ValueError("EXL3 expert weights must be loaded on the GPU")
            p.append([w.trellis.data_ptr(), w.suh.data_ptr(), w.svh.data_ptr()])
            m.append([w.padded_in, w.padded_out, w.matrix.bits_x2, w.matrix.codebook])
        ptrs.append(p)
        meta.append(m)
    return (torch.tensor(ptrs, dtype=torch.int64, device=device),
            torch.tensor(meta, dtype=torch.int64, device=device))
