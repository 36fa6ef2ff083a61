"""EXL3 checkpoint ingestion on the host.

A checkpoint directory holds safetensors files (and optionally
``model.safetensors.index.json``).  An EXL3 matrix ``<prefix>`` is the
tensor group ``<prefix>.trellis`` (int16 [K/16][N/16][8 bits_x2]),
``<prefix>.suh`` (fp16 [K]), ``<prefix>.svh`` (fp16 [N]) and exactly one
codebook marker, ``<prefix>.mcg`` or ``<prefix>.mul1``: an int32 scalar
holding that codebook's hash multiplier.  K and N are padded to whole
128-element (H128) blocks.  These are the on-disk rules the reference's
loader enforces (vllm_sm80/kernels/exl3/utils.py:183-288: inventory and
validation; quant.py:382-466: the packed weight and its H128-block shards;
quant.py:1105-1134: the expert pointer / metadata tables); the names of the
public functions and classes are the reference's, their bodies and
messages are this module's own.

Design: every file's header is parsed into ``TensorSpan`` records (absolute
byte ranges, checked to tile the payload exactly).  Tensors are grouped by
prefix in one pass and each group is classified (matrix, PLE table, or
plain tensor).  Payloads are read through read-only memory maps of the
file (numpy), so a shard copies only the tile columns and scale elements it
keeps.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

# Element sizes of the safetensors dtypes a checkpoint may hold; the FP8
# ones only in a hybrid checkpoint (tensors selected by the index).
ELEMENT_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "I16": 2, "F16": 2, "BF16": 2, "I32": 4, "F32": 4,
                 "I64": 8, "F64": 8}
FP8_ELEMENT_BYTES = {"F8_E4M3": 1, "F8_E5M2": 1, "F8_E8M0": 1}
# The dtypes this module reads as arrays.
_NUMPY = {"I16": np.int16, "F16": np.float16, "I32": np.int32}
# Codebook marker suffix -> (codebook id of the kernels, the multiplier it holds).
CODEBOOKS = {"mcg": (1, 0xCBAC1FED), "mul1": (2, 0x83DCD12D)}
_SCALE_SUFFIXES = frozenset({"suh", "svh"})
_QUANT_SUFFIXES = frozenset({"trellis"}) | _SCALE_SUFFIXES | frozenset(CODEBOOKS)
_MAX_HEADER_BYTES = 100_000_000
_BLOCK = 128   # H128 block: every padded extent and shard boundary is a multiple
_TILE = 16     # trellis tile edge


@dataclass(frozen=True)
class TensorSpan:
    """One tensor of a safetensors file: dtype, shape and its absolute byte
    range [begin, end) in ``file``."""

    name: str
    file: Path
    dtype: str
    shape: tuple
    begin: int
    end: int

    @property
    def nbytes(self) -> int:
        return self.end - self.begin

    def array(self) -> np.ndarray:
        """The payload as a read-only memory-mapped array of its shape."""
        if self.dtype not in _NUMPY:
            raise ValueError(f"{self.name}: reading {self.dtype} payloads is not supported")
        if self.nbytes == 0:
            return np.zeros(self.shape, _NUMPY[self.dtype])
        if self.shape == ():
            return np.fromfile(self.file, _NUMPY[self.dtype], count=1, offset=self.begin).reshape(())
        return np.memmap(self.file, dtype=_NUMPY[self.dtype], mode="r", offset=self.begin,
                         shape=self.shape)


def _json_object(pairs):
    """json object hook that refuses a repeated key (safetensors headers and
    the index must name each tensor once)."""
    obj = {}
    for key, value in pairs:
        if key in obj:
            raise ValueError(f"repeated JSON key {key!r}")
        obj[key] = value
    return obj


def _parse_header(path: Path):
    """(header dict, first payload byte, file size) of a safetensors file."""
    size = path.stat().st_size
    with path.open("rb") as f:
        head = f.read(8)
        if len(head) < 8:
            raise ValueError(f"{path.name}: shorter than a safetensors length prefix")
        length = int.from_bytes(head, "little")
        if length > _MAX_HEADER_BYTES or 8 + length > size:
            raise ValueError(f"{path.name}: header length {length} does not fit the file")
        header = json.loads(f.read(length), object_pairs_hook=_json_object)
    if not isinstance(header, dict):
        raise ValueError(f"{path.name}: header is not a JSON object")
    return header, 8 + length, size


def read_metadata(path) -> dict:
    """The ``__metadata__`` object of a safetensors file ({} when absent)."""
    meta = _parse_header(Path(path))[0].get("__metadata__", {})
    if not isinstance(meta, dict):
        raise ValueError(f"{Path(path).name}: __metadata__ is not a JSON object")
    return meta


def _span(path: Path, name: str, entry, payload: int, start: int, sizes: dict) -> TensorSpan:
    if not isinstance(entry, dict) or not {"dtype", "shape", "data_offsets"} <= entry.keys():
        raise ValueError(f"{path.name}: header entry {name} lacks dtype / shape / data_offsets")
    dtype, shape, offsets = entry["dtype"], entry["shape"], entry["data_offsets"]
    if dtype not in sizes:
        raise ValueError(f"{path.name}: {name} has dtype {dtype}, not one this checkpoint may hold")
    if not isinstance(shape, list) or not all(type(d) is int and d >= 0 for d in shape):
        raise ValueError(f"{path.name}: {name} has shape {shape!r}")
    if (not isinstance(offsets, list) or len(offsets) != 2
            or not all(type(v) is int for v in offsets)):
        raise ValueError(f"{path.name}: {name} has data_offsets {offsets!r}")
    lo, hi = offsets
    want = int(np.prod(shape, dtype=np.int64)) * sizes[dtype]
    if not (0 <= lo <= hi <= payload) or hi - lo != want:
        raise ValueError(f"{path.name}: {name} spans bytes [{lo}, {hi}) of a {payload}-byte payload, "
                         f"its {dtype}{shape} needs {want}")
    return TensorSpan(name, path, dtype, tuple(shape), start + lo, start + hi)


def read_headers(path, allow_fp8: bool = False) -> dict:
    """name -> TensorSpan for every tensor of one safetensors file.  Each
    span's length must match its dtype and shape, and the spans must cover
    the payload exactly: no gap, overlap or trailing byte."""
    path = Path(path)
    header, start, size = _parse_header(path)
    sizes = {**ELEMENT_BYTES, **FP8_ELEMENT_BYTES} if allow_fp8 else ELEMENT_BYTES
    payload = size - start
    spans = {name: _span(path, name, entry, payload, start, sizes)
             for name, entry in header.items() if name != "__metadata__"}
    cursor = start
    for span in sorted(spans.values(), key=lambda s: (s.begin, s.end)):
        if span.begin != cursor:
            what = "overlaps the tensor before it" if span.begin < cursor else "leaves a gap before it"
            raise ValueError(f"{path.name}: {span.name} {what}")
        cursor = span.end
    if cursor != size:
        raise ValueError(f"{path.name}: {size - cursor} payload bytes belong to no tensor")
    return spans


def admissible_rate(bits_x2: int, codebook: int) -> bool:
    """Rates the kernels and the format admit: 1..8 bits per weight in whole
    bits for either codebook, plus 1.5 / 2.5 / 3.5 bits for mul1."""
    whole = bits_x2 % 2 == 0 and 2 <= bits_x2 <= 16
    half = codebook == CODEBOOKS["mul1"][0] and bits_x2 in (3, 5, 7)
    return whole or half


@dataclass(frozen=True)
class PackedMatrix:
    """A validated EXL3 matrix of the checkpoint (padded geometry, rate,
    codebook and the marker suffix it was stored with)."""

    prefix: str
    padded_in: int
    padded_out: int
    bits_x2: int
    codebook: int
    marker: str

    @property
    def keys(self) -> tuple:
        return (f"{self.prefix}.trellis", f"{self.prefix}.suh", f"{self.prefix}.svh",
                f"{self.prefix}.{self.marker}")

    def validate_logical(self, logical_in: int, logical_out: int) -> None:
        """The logical sizes must pad to exactly the stored blocks."""
        for logical, padded, side in ((logical_in, self.padded_in, "input"),
                                      (logical_out, self.padded_out, "output")):
            if logical <= 0 or -(-logical // _BLOCK) * _BLOCK != padded:
                raise ValueError(f"{self.prefix}: logical {side} size {logical} does not pad to "
                                 f"the stored {padded}")


def _classify(prefix: str, parts: dict) -> PackedMatrix:
    """The PackedMatrix of a tensor group holding a trellis, or ValueError."""
    trellis = parts["trellis"]
    if trellis.dtype != "I16" or len(trellis.shape) != 3:
        raise ValueError(f"{prefix}.trellis must be int16 [K/16][N/16][words], "
                         f"not {trellis.dtype}{list(trellis.shape)}")
    k, n, words = trellis.shape[0] * _TILE, trellis.shape[1] * _TILE, trellis.shape[2]
    if k == 0 or n == 0 or k % _BLOCK or n % _BLOCK or words == 0 or words % 8:
        raise ValueError(f"{prefix}: trellis of {k} x {n} weights with {words} words per tile is "
                         "not whole H128 blocks of whole 16 x 16 tiles")
    for suffix, length in (("suh", k), ("svh", n)):
        scale = parts.get(suffix)
        if scale is None or scale.dtype != "F16" or scale.shape != (length,):
            raise ValueError(f"{prefix}.{suffix} must be fp16 [{length}]")
    markers = sorted(CODEBOOKS.keys() & parts.keys())
    if len(markers) != 1:
        raise ValueError(f"{prefix}: needs exactly one codebook marker (.mcg or .mul1), found "
                         f"{len(markers)}")
    marker = markers[0]
    codebook, multiplier = CODEBOOKS[marker]
    span = parts[marker]
    if span.dtype != "I32" or span.shape != ():
        raise ValueError(f"{prefix}.{marker} must be an int32 scalar")
    stored = int(span.array().astype(np.uint32))
    if stored != multiplier:
        raise ValueError(f"{prefix}.{marker} holds multiplier {stored:#010x}, that codebook's is "
                         f"{multiplier:#010x}")
    bits_x2 = words // 8
    if not admissible_rate(bits_x2, codebook):
        raise ValueError(f"{prefix}: {bits_x2 / 2:g} bits per weight is not a rate of codebook "
                         f"{marker}")
    if "weight" in parts:
        raise ValueError(f"{prefix} holds both a dense .weight and an EXL3 trellis")
    return PackedMatrix(prefix, k, n, bits_x2, codebook, marker)


def _weight_map(directory: Path, required: bool):
    index = directory / "model.safetensors.index.json"
    if not index.exists():
        if required:
            raise ValueError(f"{directory}: selecting tensors by index needs "
                             "model.safetensors.index.json")
        return None
    data = json.loads(index.read_text(), object_pairs_hook=_json_object)
    weight_map = data.get("weight_map") if isinstance(data, dict) else None
    if not isinstance(weight_map, dict):
        raise ValueError(f"{index.name}: no weight_map object")
    return weight_map


class Exl3Manifest:
    """Inventory of an EXL3 checkpoint directory.

    ``tensors``: name -> TensorSpan over every ``*.safetensors`` file (with
    ``select_by_index``, a hybrid checkpoint: only the tensors the index
    assigns to the file holding them; ``unselected`` counts the others).
    ``matrices``: prefix -> PackedMatrix.  ``ple_tables``: prefix ->
    TensorSpan of the row-decoded embedding tables (``*.ngram_embedding``
    trellises, read by the PLE row decoder, not by the linear kernels)."""

    def __init__(self, directory, select_by_index: bool = False):
        self.directory = Path(directory)
        files = sorted(self.directory.glob("*.safetensors"))
        if not files:
            raise ValueError(f"{self.directory}: no *.safetensors files (EXL3 loads local "
                             "checkpoints only)")
        weight_map = _weight_map(self.directory, select_by_index)
        self.tensors: dict = {}
        self.unselected = 0
        for path in files:
            for name, span in read_headers(path, allow_fp8=select_by_index).items():
                if select_by_index and weight_map.get(name) != path.name:
                    self.unselected += 1
                elif name in self.tensors:
                    raise ValueError(f"tensor {name} appears in both {self.tensors[name].file.name} "
                                     f"and {path.name}")
                else:
                    self.tensors[name] = span
        self.tensors = dict(sorted(self.tensors.items()))
        for name, filename in (weight_map or {}).items():
            span = self.tensors.get(name)
            if span is None or span.file.name != filename:
                raise ValueError(f"the index puts {name} in {filename}, which does not hold it")
        groups: dict = {}
        for name, span in self.tensors.items():
            prefix, _, suffix = name.rpartition(".")
            groups.setdefault(prefix, {})[suffix] = span
        self.matrices: dict = {}
        self.ple_tables: dict = {}
        for prefix, parts in groups.items():
            quant = _QUANT_SUFFIXES & parts.keys()
            if not quant:
                continue
            if "trellis" not in parts:
                if not any(prefix.startswith(p + ".") for p in groups
                           if p.endswith(".ngram_embedding") and "trellis" in groups[p]):
                    raise ValueError(f"{prefix}: EXL3 tensors {sorted(quant)} without a trellis")
                continue
            if prefix.endswith(".ngram_embedding"):
                self.ple_tables[prefix] = parts["trellis"]
                continue
            self.matrices[prefix] = _classify(prefix, parts)

    def expect(self, name: str, dtype: str, shape: tuple) -> TensorSpan:
        """The tensor ``name``, which must exist with this dtype and shape."""
        span = self.tensors.get(name)
        if span is None or span.dtype != dtype or span.shape != tuple(shape):
            found = "absent" if span is None else f"{span.dtype}{list(span.shape)}"
            raise ValueError(f"{name}: expected {dtype}{list(shape)}, found {found}")
        return span


# ---- H128-block shards -------------------------------------------------------------

def _check_rank(rank: int, size: int, rotation: int = 0) -> None:
    if size < 1 or not 0 <= rank < size or rotation < 0:
        raise ValueError(f"shard rank {rank} of {size} (rotation {rotation}) is not a shard")


def aligned_shard(logical: int, padded: int, rank: int, size: int) -> slice:
    """Rank ``rank`` of ``size`` equal shards, each whole H128 blocks (one
    rank keeps the whole padded extent)."""
    _check_rank(rank, size)
    if size == 1:
        return slice(0, padded)
    per_rank, rest = divmod(logical, size)
    if logical != padded or rest or per_rank == 0 or per_rank % _BLOCK:
        raise ValueError(f"{logical} elements (padded {padded}) do not split into {size} equal "
                         "shards of whole H128 blocks")
    return slice(rank * per_rank, (rank + 1) * per_rank)


def block_shard(logical: int, padded: int, rank: int, size: int, rotation: int = 0) -> slice:
    """Whole H128 blocks dealt to ``size`` chunks as evenly as they go (the
    first ``blocks % size`` chunks hold one block more); rank ``rank`` takes
    chunk ``(rank + rotation) % size``."""
    _check_rank(rank, size, rotation)
    if size == 1:
        return slice(0, padded)
    if logical != padded or logical % _BLOCK:
        raise ValueError(f"{logical} elements (padded {padded}) are not whole H128 blocks")
    blocks = logical // _BLOCK
    if blocks < size:
        raise ValueError(f"{blocks} H128 blocks cannot give each of {size} ranks one")
    counts = [blocks // size + (chunk < blocks % size) for chunk in range(size)]
    chunk = (rank + rotation) % size
    first = sum(counts[:chunk])
    return slice(first * _BLOCK, (first + counts[chunk]) * _BLOCK)


def _block_extent(part: slice, limit: int) -> int:
    if (part.step not in (None, 1) or part.start is None or part.stop is None
            or not 0 <= part.start < part.stop <= limit or part.start % _BLOCK or part.stop % _BLOCK):
        raise ValueError(f"shard {part} of an extent of {limit} is not whole H128 blocks")
    return part.stop - part.start


class Exl3PackedWeight:
    """A matrix, or a shard of it: one input range and one or more output
    ranges, each whole H128 blocks.  After ``load``: trellis int16
    [padded_in / 16][padded_out / 16][8 bits_x2] (the output ranges' tile
    columns side by side), suh fp16 [padded_in], svh fp16 [padded_out]."""

    def __init__(self, matrix: PackedMatrix, logical_in: int, logical_out: int,
                 input_slice: slice, output_slices: list):
        self.matrix = matrix
        self.input_slice = input_slice
        self.output_slices = list(output_slices)
        if not self.output_slices:
            raise ValueError(f"{matrix.prefix}: a shard needs an output range")
        self.padded_in = _block_extent(input_slice, matrix.padded_in)
        self.padded_out = sum(_block_extent(p, matrix.padded_out) for p in self.output_slices)
        if not (0 < logical_in <= self.padded_in and 0 < logical_out <= self.padded_out):
            raise ValueError(f"{matrix.prefix}: logical {logical_in} x {logical_out} exceeds the "
                             f"shard's {self.padded_in} x {self.padded_out}")
        self.logical_in = logical_in
        self.logical_out = logical_out
        self.trellis = self.suh = self.svh = None
        self.loaded = False

    def load(self, manifest: Exl3Manifest) -> None:
        """Copies the shard's tile columns and scale elements out of the
        checkpoint's memory-mapped payloads."""
        prefix = self.matrix.prefix
        rows = slice(self.input_slice.start // _TILE, self.input_slice.stop // _TILE)
        tiles = manifest.tensors[f"{prefix}.trellis"].array()[rows]
        self.trellis = torch.from_numpy(np.concatenate(
            [tiles[:, p.start // _TILE:p.stop // _TILE] for p in self.output_slices], axis=1))
        self.suh = torch.from_numpy(np.array(manifest.tensors[f"{prefix}.suh"].array()[self.input_slice]))
        svh = manifest.tensors[f"{prefix}.svh"].array()
        self.svh = torch.from_numpy(np.concatenate([svh[p] for p in self.output_slices]))
        self.loaded = True

    def to(self, device) -> "Exl3PackedWeight":
        if not self.loaded:
            raise ValueError(f"{self.matrix.prefix}: load the weight before moving it")
        self.trellis, self.suh, self.svh = (t.to(device) for t in (self.trellis, self.suh, self.svh))
        return self


def load_matrix(manifest: Exl3Manifest, prefix: str, logical_in: int, logical_out: int,
                device=None) -> Exl3PackedWeight:
    """The whole matrix ``prefix`` (one GPU, no shard), its logical geometry
    checked, loaded (and moved to ``device``)."""
    matrix = manifest.matrices.get(prefix)
    if matrix is None:
        raise ValueError(f"the checkpoint has no EXL3 matrix {prefix}")
    matrix.validate_logical(logical_in, logical_out)
    weight = Exl3PackedWeight(matrix, logical_in, logical_out, slice(0, matrix.padded_in),
                              [slice(0, matrix.padded_out)])
    weight.load(manifest)
    return weight.to(device) if device is not None else weight


def expert_tables(experts, device) -> tuple:
    """(packed_ptrs int64 [E][3][3], packed_meta int64 [E][3][4]) of loaded
    expert weights [E][gate, up, down] on the device: each projection's
    trellis / suh / svh addresses, and its padded_in, padded_out, bits_x2,
    codebook (the tables the MoE kernels read)."""
    ptrs = np.zeros((len(experts), 3, 3), np.int64)
    meta = np.zeros((len(experts), 3, 4), np.int64)
    for e, projections in enumerate(experts):
        if len(projections) != 3:
            raise ValueError(f"expert {e} has {len(projections)} projections, not gate / up / down")
        for p, w in enumerate(projections):
            if not w.loaded or not all(t.is_cuda for t in (w.trellis, w.suh, w.svh)):
                raise ValueError(f"expert {e} projection {p} is not loaded on the GPU")
            ptrs[e, p] = (w.trellis.data_ptr(), w.suh.data_ptr(), w.svh.data_ptr())
            meta[e, p] = (w.padded_in, w.padded_out, w.matrix.bits_x2, w.matrix.codebook)
    return torch.from_numpy(ptrs).to(device), torch.from_numpy(meta).to(device)
