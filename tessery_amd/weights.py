"""Weight packs on disk: verified artifact reads and a SafeTensors parser that executes nothing.

Mirrors tessery's weights.py (read_artifact :23-51, read_json :54-64, SafeTensors :75-133) and
files.directory (files.py:12-23): the same acceptance rules and the same ManifestError on every
rejection, so a pack tessery accepts loads here unchanged and a pack it refuses is refused here.
The bytes are read once, hashed, and every GPU upload is a view of that verified snapshot.
"""

from __future__ import annotations

import hashlib
import json
import math
import os
import stat
import struct
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterator, Mapping

import numpy as np
from numpy.typing import NDArray

from .errors import ManifestError

# Bytes per element of the dtypes a pack may hold (weights.py:98-110).
DTYPE_WIDTH = {"BF16": 2, "U32": 4, "F32": 4, "I64": 8}
HEADER_LIMIT = 4 * 1024 * 1024
JSON_LIMIT = 16 * 1024 * 1024


def _unique_pairs(pairs: list[tuple[str, Any]]) -> dict[str, Any]:
    result: dict[str, Any] = {}
    for key, value in pairs:
        if key in result:
            raise ValueError("duplicate key")
        result[key] = value
    return result


def _no_constant(_: str) -> Any:
    raise ValueError("NaN and Infinity are not JSON")


def _finite_float(text: str) -> float:
    value = float(text)
    if not math.isfinite(value):
        raise ValueError("float out of range")
    return value


def strict_json(data: bytes, *, limit: int) -> Any:
    """RFC JSON only (json_codec.py:30-41): UTF-8, no duplicate keys, no NaN/Infinity, finite
    floats, at most limit bytes. Raises ManifestError otherwise."""
    if len(data) > limit:
        raise ManifestError()
    try:
        return json.loads(data.decode("utf-8"), object_pairs_hook=_unique_pairs,
                          parse_constant=_no_constant, parse_float=_finite_float)
    except (ValueError, RecursionError):
        raise ManifestError() from None


@contextmanager
def directory(path: str) -> Iterator[int]:
    """A descriptor of an absolute directory path opened component by component without following
    symlinks; '.' and '..' components are refused (files.py:12-23)."""
    if not isinstance(path, str) or not path.startswith("/") or any(
            part in {".", ".."} for part in path.split("/")):
        raise ManifestError()
    try:
        fd = os.open("/", os.O_RDONLY | os.O_DIRECTORY)
    except OSError:
        raise ManifestError() from None
    try:
        for part in Path(path).parts[1:]:
            child = os.open(part, os.O_RDONLY | os.O_DIRECTORY | os.O_NOFOLLOW, dir_fd=fd)
            os.close(fd)
            fd = child
        yield fd
    except OSError:
        raise ManifestError() from None
    finally:
        os.close(fd)


@dataclass(frozen=True)
class Artifact:
    """One pinned file of a pack: its name in the pack, file name, exact size and sha256."""

    name: str
    filename: str
    size: int
    sha256: str


def read_artifact(model_dir: str, artifact: Artifact) -> bytes:
    """The file's bytes, after a no-follow open of a regular file with one link and exactly the
    pinned size, whose sha256 matches (weights.py:23-51). Other files in the directory are never
    read."""
    try:
        with directory(model_dir) as dir_fd:
            fd = os.open(artifact.filename, os.O_RDONLY | os.O_NOFOLLOW | os.O_NONBLOCK,
                         dir_fd=dir_fd)
            with os.fdopen(fd, "rb") as stream:
                info = os.fstat(stream.fileno())
                if (not stat.S_ISREG(info.st_mode) or info.st_nlink != 1
                        or info.st_size != artifact.size):
                    raise ManifestError()
                data = stream.read(artifact.size + 1)
        if len(data) != artifact.size or hashlib.sha256(data).hexdigest() != artifact.sha256:
            raise ManifestError()
        return data
    except (OSError, ValueError):
        raise ManifestError() from None


def read_json(model_dir: str, artifact: Artifact) -> dict[str, Any]:
    value = strict_json(read_artifact(model_dir, artifact), limit=JSON_LIMIT)
    if not isinstance(value, dict):
        raise ManifestError()
    return value


@dataclass(frozen=True)
class TensorInfo:
    dtype: str
    shape: tuple[int, ...]
    start: int
    end: int


class SafeTensors:
    """A parsed SafeTensors byte snapshot (weights.py:75-133). Accepted only when:

    - the 8-byte little-endian header length is in (0, 4 MiB] and fits the data;
    - the header is a strict JSON object; "__metadata__" is skipped;
    - every tensor record has exactly dtype, shape and data_offsets, dtype in BF16/U32/F32/I64,
      a rank 1 or 2 shape of ints in [1, 200000], and offsets [start, end) inside the payload
      with end - start = elements * width;
    - the tensors tile the payload exactly, in offset order, with no gap or overlap.
    """

    def __init__(self, data: bytes) -> None:
        self.data = data
        if len(data) < 8:
            raise ManifestError()
        length = struct.unpack_from("<Q", data)[0]
        if not 0 < length <= HEADER_LIMIT or length + 8 > len(data):
            raise ManifestError()
        header = strict_json(data[8:8 + length], limit=HEADER_LIMIT)
        if not isinstance(header, dict):
            raise ManifestError()
        self.base = length + 8
        payload = len(data) - self.base
        self.tensors: dict[str, TensorInfo] = {}
        for name, item in header.items():
            if name == "__metadata__":
                continue
            if not isinstance(item, dict) or set(item) != {"dtype", "shape", "data_offsets"}:
                raise ManifestError()
            dtype, shape, offsets = item["dtype"], item["shape"], item["data_offsets"]
            if (not isinstance(dtype, str) or dtype not in DTYPE_WIDTH
                    or not isinstance(shape, list) or not 1 <= len(shape) <= 2
                    or any(type(d) is not int or not 0 < d <= 200000 for d in shape)
                    or not isinstance(offsets, list) or len(offsets) != 2
                    or any(type(d) is not int for d in offsets)):
                raise ManifestError()
            start, end = offsets
            if not 0 <= start < end <= payload or end - start != math.prod(shape) * DTYPE_WIDTH[dtype]:
                raise ManifestError()
            self.tensors[name] = TensorInfo(dtype, tuple(shape), start, end)
        cursor = 0
        for info in sorted(self.tensors.values(), key=lambda t: t.start):
            if info.start != cursor:
                raise ManifestError()
            cursor = info.end
        if cursor != payload:
            raise ManifestError()

    def view(self, name: str, *, shape: tuple[int, ...], dtype: str) -> NDArray[np.uint8]:
        """The raw bytes of tensor name, which must have exactly this shape and dtype."""
        info = self.tensors.get(name)
        if info is None or info.shape != shape or info.dtype != dtype:
            raise ManifestError()
        return np.frombuffer(self.data, dtype=np.uint8, count=info.end - info.start,
                             offset=self.base + info.start)


_NUMPY_OF = {"BF16": np.uint16, "U32": np.uint32, "F32": np.float32, "I64": np.int64}


def encode_safetensors(tensors: Mapping[str, tuple[str, NDArray[Any]]]) -> bytes:
    """SafeTensors bytes for name -> (dtype, array); BF16 arrays are given as their uint16 words.
    Tensors are laid out in name order; the header is padded with spaces to 8 bytes. Used to write
    synthetic packs of the real model shapes (no real weights are needed to exercise the path)."""
    header: dict[str, Any] = {}
    chunks = []
    offset = 0
    for name in sorted(tensors):
        dtype, array = tensors[name]
        raw = np.ascontiguousarray(array, dtype=_NUMPY_OF[dtype]).tobytes()
        header[name] = {"dtype": dtype, "shape": list(np.shape(array)),
                        "data_offsets": [offset, offset + len(raw)]}
        chunks.append(raw)
        offset += len(raw)
    encoded = json.dumps(header, separators=(",", ":")).encode()
    encoded += b" " * (-len(encoded) % 8)
    return struct.pack("<Q", len(encoded)) + encoded + b"".join(chunks)


def artifact_of(name: str, filename: str, data: bytes) -> Artifact:
    return Artifact(name, filename, len(data), hashlib.sha256(data).hexdigest())
