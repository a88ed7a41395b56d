"""Persistent artifacts: PSCLS100 checkpoints (crates/leo-format/src/lib.rs)
and LEODATA1 prepared datasets (crates/leo-data/src/lib.rs), over the host
artifact layer of libleo_hip.so (include/leo_formats.h).

The function names and behaviour follow the reference crates: a checkpoint is
written to ``path.tmp``, synced and renamed into place; committing bumps the
model's generation and keeps older generations as ``path.genNNNNNN``; loading
validates every structural rule, digest and the semantics contract before a
Model is returned. Errors are ``native.LeoError`` with ``code`` ERR_CORRUPT,
ERR_INCOMPATIBLE or ERR_IO (LeoError::checkpoint_corrupt / _incompatible / io).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

from . import native
from .config import Config
from .model import Model, host_config

PathLike = Union[str, os.PathLike]
MAX_CHECKPOINT_BYTES = 64 * 1024 * 1024 * 1024  # lib.rs:27


def _lib() -> ctypes.CDLL:
    return native.load()


def _path(p: PathLike) -> bytes:
    return os.fsencode(os.fspath(p))


def _digest(d: native.LeoDigest) -> bytes:
    return bytes(d.bytes)


def _as_digest(b: bytes) -> native.LeoDigest:
    if len(b) != 32:
        raise ValueError("a SHA-256 digest is 32 bytes")
    d = native.LeoDigest()
    ctypes.memmove(d.bytes, b, 32)
    return d


# --- digests (crates/leo-core/src/artifact.rs) -------------------------------
def digest_bytes(data: bytes) -> bytes:
    lib = _lib()
    out = native.LeoDigest()
    buf = np.frombuffer(bytes(data), dtype=np.uint8)
    native.check(lib, lib.leo_sha256(buf.ctypes.data if buf.size else None, buf.size, ctypes.byref(out)))
    return _digest(out)


def digest_file(path: PathLike) -> bytes:
    lib = _lib()
    out = native.LeoDigest()
    native.check(lib, lib.leo_sha256_file(_path(path), ctypes.byref(out)))
    return _digest(out)


# --- PSCLS100 checkpoints -------------------------------------------------------
def encode_model(model: Model) -> bytes:
    """encode_model (lib.rs:289-444); the model is validated first."""
    lib = _lib()
    hc = host_config(model.config)
    view = model.view()
    text = model.config.to_toml().encode()
    size = ctypes.c_uint64(0)
    native.check(lib, lib.leo_checkpoint_encoded_size(ctypes.byref(hc), len(text), ctypes.byref(size)))
    out = np.zeros(size.value, dtype=np.uint8)
    native.check(lib, lib.leo_checkpoint_encode(ctypes.byref(hc), ctypes.byref(view), text, len(text),
                                                out.ctypes.data, out.size))
    return out.tobytes()


def decode_model(data: bytes) -> Model:
    """decode_model (lib.rs:446-620): structure and digests, the CONFIG text
    (parsed and validated as Config::from_toml does), then the tensors."""
    lib = _lib()
    buf = np.frombuffer(bytes(data), dtype=np.uint8)
    ptr = buf.ctypes.data if buf.size else None
    info = native.LeoCheckpointInfo()
    native.check(lib, lib.leo_checkpoint_inspect(ptr, buf.size, ctypes.byref(info)))
    text = buf[info.config_offset:info.config_offset + info.config_length].tobytes()
    try:
        config = Config.from_toml(text.decode("utf-8"))
    except UnicodeDecodeError as error:
        raise native.LeoError(native.ERR_CORRUPT, f"invalid CONFIG UTF-8: {error}") from None
    model = Model.empty(config)
    hc = host_config(config)
    view = model.view()
    native.check(lib, lib.leo_checkpoint_decode(ptr, buf.size, ctypes.byref(hc), ctypes.byref(view)))
    model._absorb(view)
    return model


def save_model_atomic(path: PathLike, model: Model, retain_previous: bool) -> None:
    """save_model_atomic (lib.rs:144-175)."""
    lib = _lib()
    hc = host_config(model.config)
    view = model.view()
    text = model.config.to_toml().encode()
    native.check(lib, lib.leo_checkpoint_save_atomic(_path(path), ctypes.byref(hc), ctypes.byref(view), text,
                                                     len(text), 1 if retain_previous else 0))


def commit_model(path: PathLike, model: Model) -> None:
    """commit_model (lib.rs:177-185): generation + 1, keeping the previous
    checkpoint as a generation file; the generation is restored on failure."""
    previous = model.generation
    model.generation = previous + 1
    try:
        save_model_atomic(path, model, True)
    except BaseException:
        model.generation = previous
        raise


def commit_model_rolling(path: PathLike, model: Model, keep_previous_generations: int) -> None:
    """commit_model_rolling (lib.rs:187-199)."""
    previous = model.generation
    model.generation = previous + 1
    try:
        save_model_atomic(path, model, keep_previous_generations > 0)
    except BaseException:
        model.generation = previous
        raise
    lib = _lib()
    native.check(lib, lib.leo_checkpoint_prune_generations(_path(path), keep_previous_generations))


def load_model(path: PathLike) -> Model:
    """load_model (lib.rs:241-251)."""
    length = os.stat(path).st_size
    if length > MAX_CHECKPOINT_BYTES:
        raise native.LeoError(native.ERR_CORRUPT, f"checkpoint is too large: {length} bytes")
    with open(path, "rb") as f:
        return decode_model(f.read())


def generation_path(path: PathLike, generation: int) -> str:
    """generation_path (lib.rs:276-278)."""
    return f"{os.fspath(path)}.gen{generation:06d}"


def rollback_model(path: PathLike, generation: int) -> Model:
    """rollback_model (lib.rs:253-256 + 265-274): loads generation `generation`
    and saves it as the current checkpoint (keeping the current one)."""
    source = generation_path(path, generation)
    if not os.path.exists(source):
        raise native.LeoError(native.ERR_CORRUPT, f"generation {generation} not found at {source}")
    model = load_model(source)
    save_model_atomic(path, model, True)
    return model


def read_generation(path: PathLike) -> int:
    """read_generation (lib.rs:258-264)."""
    lib = _lib()
    out = ctypes.c_uint64(0)
    native.check(lib, lib.leo_checkpoint_read_generation(_path(path), ctypes.byref(out)))
    return out.value


def checkpoint_hash(path: PathLike) -> bytes:
    """checkpoint_hash (lib.rs:266-268): SHA-256 of the checkpoint file."""
    return digest_file(path)


checkpoint_digest = checkpoint_hash


# --- LEODATA1 prepared datasets -------------------------------------------------
@dataclass(frozen=True)
class StoryIndex:
    """StoryIndex (lib.rs:22-27)."""

    offset: int
    length: int
    split_flags: int = 0


@dataclass(frozen=True)
class DatasetIdentity:
    """DatasetIdentity (lib.rs:29-38)."""

    schema_version: int
    record_count: int
    bytes_length: int
    bytes_digest: bytes
    records_digest: bytes
    provenance_digest: bytes
    dataset_id: bytes

    @classmethod
    def from_c(cls, c: native.LeoDatasetIdentity) -> "DatasetIdentity":
        return cls(int(c.schema_version), int(c.record_count), int(c.bytes_length), _digest(c.bytes_digest),
                   _digest(c.records_digest), _digest(c.provenance_digest), _digest(c.dataset_id))


def compute_dataset_id(schema_version: int, record_count: int, bytes_length: int, bytes_digest: bytes,
                       records_digest: bytes, provenance_digest: bytes) -> bytes:
    """compute_dataset_id (lib.rs:237-253)."""
    lib = _lib()
    out = native.LeoDigest()
    args = [_as_digest(bytes_digest), _as_digest(records_digest), _as_digest(provenance_digest)]
    native.check(lib, lib.leo_dataset_compute_id(schema_version, record_count, bytes_length,
                                                 *[ctypes.byref(a) for a in args], ctypes.byref(out)))
    return _digest(out)


def write_index(index_path: PathLike, bytes_path: PathLike, entries: Sequence[StoryIndex],
                provenance_digest: bytes) -> DatasetIdentity:
    """write_index (lib.rs:255-323)."""
    lib = _lib()
    table = (native.LeoStoryIndex * max(len(entries), 1))()
    for i, e in enumerate(entries):
        table[i] = native.LeoStoryIndex(e.offset, e.length, e.split_flags)
    prov = _as_digest(provenance_digest)
    out = native.LeoDatasetIdentity()
    native.check(lib, lib.leo_dataset_write_index(_path(index_path), _path(bytes_path), table, len(entries),
                                                  ctypes.byref(prov), ctypes.byref(out)))
    return DatasetIdentity.from_c(out)


class PreparedDataset:
    """PreparedDataset (lib.rs:40-229): opening validates the whole artifact
    pair; stories are read by offset and checked to be UTF-8."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def open(cls, bytes_path: PathLike, index_path: PathLike) -> "PreparedDataset":
        lib = _lib()
        out = ctypes.c_void_p()
        native.check(lib, lib.leo_dataset_open(_path(bytes_path), _path(index_path), ctypes.byref(out)))
        return cls(out.value)

    def close(self) -> None:
        if self._h:
            _lib().leo_dataset_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self) -> "PreparedDataset":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def identity(self) -> DatasetIdentity:
        lib = _lib()
        out = native.LeoDatasetIdentity()
        native.check(lib, lib.leo_dataset_identity(self._h, ctypes.byref(out)))
        return DatasetIdentity.from_c(out)

    def __len__(self) -> int:
        return int(_lib().leo_dataset_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    def entry(self, index: int) -> Optional[StoryIndex]:
        if not 0 <= index < len(self):
            return None
        lib = _lib()
        out = native.LeoStoryIndex()
        native.check(lib, lib.leo_dataset_entry(self._h, index, ctypes.byref(out)))
        return StoryIndex(int(out.offset), int(out.length), int(out.split_flags))

    def story(self, index: int) -> bytes:
        lib = _lib()
        entry = self.entry(index)
        if entry is None:
            raise native.LeoError(native.ERR_INVALID_ARGUMENT, "story index out of range")
        buf = np.zeros(max(entry.length, 1), dtype=np.uint8)
        n = ctypes.c_uint64(0)
        native.check(lib, lib.leo_dataset_story(self._h, index, buf.ctypes.data, buf.size, ctypes.byref(n)))
        return buf[:n.value].tobytes()

    def pack(self, first: int, count: int) -> Tuple[np.ndarray, np.ndarray]:
        """Stories [first, first+count) as (bytes, offsets) for train_batch / evaluate."""
        lib = _lib()
        offsets = np.zeros(count + 1, dtype=np.uint64)
        native.check(lib, lib.leo_dataset_pack(self._h, first, count, None, 0, offsets.ctypes.data))
        data = np.zeros(max(int(offsets[-1]), 1), dtype=np.uint8)
        native.check(lib, lib.leo_dataset_pack(self._h, first, count, data.ctypes.data, data.size,
                                               offsets.ctypes.data))
        return data[:int(offsets[-1])], offsets

    def stories(self, first: int, count: int) -> List[bytes]:
        data, offsets = self.pack(first, count)
        return [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(count)]
