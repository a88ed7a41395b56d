"""The host artifact layer (include/leo_formats.h, leo_amd/formats.py) on the CPU.

* SHA-256 against hashlib and the FIPS 180-4 examples;
* PSCLS100: the reference's own checkpoint tests restated with their literals
  (crates/leo-format/tests/checkpoint.rs:8-97 and the unit tests of
  crates/leo-format/src/lib.rs:1178-1228), the byte layout read back with
  ``struct`` straight from the reference's field table (lib.rs:20-28, 413-444,
  810-827), and a trained model round trip;
* LEODATA1: the reference's tests (crates/leo-data/src/lib.rs:331-400), an
  index written independently with ``struct``/hashlib in the layout of
  python/prepare_tinystories.py:200-262 (byte-identical to ours, and opened by
  our reader), and the rejection rules of PreparedDataset::open.
"""
from __future__ import annotations

import hashlib
import os
import struct

import numpy as np
import pytest

from leo_amd import formats, native
from leo_amd.model import ARRAY_FIELDS, Model
from tests.helpers import toml_test_config

HEADER, DESCRIPTOR, ALIGN = 128, 128, 64


def _sha(b: bytes) -> bytes:
    return hashlib.sha256(b).digest()


# --- SHA-256 -------------------------------------------------------------------
def test_sha256_matches_fips_examples_and_hashlib(tmp_path):
    assert formats.digest_bytes(b"abc").hex() == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert formats.digest_bytes(b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert formats.digest_bytes(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    rng = np.random.default_rng(3)
    for n in (1, 55, 56, 57, 63, 64, 65, 119, 120, 128, 1000, 65537):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert formats.digest_bytes(data) == _sha(data), n
    data = rng.integers(0, 256, (1 << 21) + 13, dtype=np.uint8).tobytes()
    path = tmp_path / "blob"
    path.write_bytes(data)
    assert formats.digest_file(path) == _sha(data)


# --- PSCLS100 ---------------------------------------------------------------------
def _model() -> Model:
    return Model.initialize(toml_test_config())


def _equal(a: Model, b: Model) -> bool:
    return all(np.array_equal(getattr(a, k), getattr(b, k)) for k in ARRAY_FIELDS) and \
        a.generation == b.generation and a.parameter_revision == b.parameter_revision and \
        a.statistics == b.statistics and a.config == b.config


def test_checkpoint_round_trip_preserves_tensors(tmp_path):
    # checkpoint.rs:8-38
    model = _model()
    model.parameter_revision = 23
    model.statistics["persistent_ticks"] = 17
    model.statistics["active_neurons_sum"] = 51
    model.in_weight[0] = 0.75
    model.ctx_keys[0] = 42
    model.ctx_emb[0] = 0.5
    model.ctx_out[0] = -0.25
    model.ctx_obs[0] = 7
    path = tmp_path / "roundtrip.pscls"
    formats.save_model_atomic(path, model, False)
    before = formats.checkpoint_hash(path)
    loaded = formats.load_model(path)
    assert loaded.generation == model.generation and loaded.parameter_revision == 23
    assert np.array_equal(loaded.rec_target, model.rec_target)
    assert np.array_equal(loaded.out_weight, model.out_weight)
    assert np.array_equal(loaded.in_weight, model.in_weight)
    for k in ("ctx_keys", "ctx_emb", "ctx_out", "ctx_obs"):
        assert np.array_equal(getattr(loaded, k), getattr(model, k)), k
    assert loaded.statistics["persistent_ticks"] == 17
    assert loaded.statistics["active_neurons_sum"] / loaded.statistics["persistent_ticks"] == 3.0
    assert formats.checkpoint_hash(path) == before
    assert before == _sha(path.read_bytes())
    assert _equal(loaded, model)
    assert not (tmp_path / "roundtrip.pscls.tmp").exists()


def test_rolling_checkpoint_keeps_only_current_and_previous_model(tmp_path):
    # checkpoint.rs:40-62
    model = _model()
    path = tmp_path / "rolling.pscls"
    formats.save_model_atomic(path, model, False)
    for revision in range(1, 5):
        model.parameter_revision = revision
        formats.commit_model_rolling(path, model, 1)
    assert formats.load_model(path).generation == 4
    assert formats.load_model(path).parameter_revision == 4
    assert formats.read_generation(path) == 4
    for g in (0, 1, 2):
        assert not os.path.exists(formats.generation_path(path, g))
    assert os.path.exists(formats.generation_path(path, 3))
    assert formats.generation_path(path, 3).endswith(".gen000003")


def test_commit_keeps_generations_and_rollback_restores_one(tmp_path):
    # commit_model (lib.rs:177-185), rollback_model (lib.rs:253-256)
    model = _model()
    path = tmp_path / "ckpt" / "model.pscls"  # the parent directory is created
    formats.save_model_atomic(path, model, False)
    first = model.copy()
    model.threshold[:] = np.float32(0.3)
    formats.commit_model(path, model)
    assert model.generation == 1 and formats.read_generation(path) == 1
    assert os.path.exists(formats.generation_path(path, 0))
    restored = formats.rollback_model(path, 0)
    assert _equal(restored, first)
    assert formats.read_generation(path) == 0
    assert os.path.exists(formats.generation_path(path, 1))  # the replaced checkpoint is kept
    with pytest.raises(native.LeoError) as e:
        formats.rollback_model(path, 7)
    assert e.value.code == native.ERR_CORRUPT


def test_failed_commit_restores_the_generation(tmp_path):
    model = _model()
    model.threshold[0] = np.float32(5.0)  # outside the canonical bounds: validation fails
    with pytest.raises(native.LeoError):
        formats.commit_model(tmp_path / "bad.pscls", model)
    assert model.generation == 0 and not (tmp_path / "bad.pscls").exists()


def test_corrupted_checkpoint_is_rejected():
    # checkpoint.rs:81-93
    data = bytearray(formats.encode_model(_model()))
    data[32] ^= 0xFF
    with pytest.raises(native.LeoError) as e:
        formats.decode_model(bytes(data))
    assert e.value.code == native.ERR_CORRUPT


def _resign(data: bytearray) -> bytes:
    """Recomputes every section digest and the header digest (lib.rs:413-444),
    so that a structural change is what a decoder sees."""
    count = struct.unpack_from("<I", data, 24)[0]
    for i in range(count):
        d = HEADER + i * DESCRIPTOR
        offset, length = struct.unpack_from("<QQ", data, d + 48)
        data[d + 72:d + 104] = _sha(bytes(data[offset:offset + length]))
    data[96:128] = bytes(32)
    data[96:128] = _sha(bytes(data[:HEADER]))
    return bytes(data)


def _descriptor(data: bytes, kind: int):
    for i in range(struct.unpack_from("<I", data, 24)[0]):
        d = HEADER + i * DESCRIPTOR
        if struct.unpack_from("<I", data, d)[0] == kind:
            return d
    raise KeyError(kind)


def test_duplicate_section_descriptors_are_rejected():
    # lib.rs:1192-1199
    data = bytearray(formats.encode_model(_model()))
    data[HEADER + DESCRIPTOR:HEADER + DESCRIPTOR + 4] = data[HEADER:HEADER + 4]
    with pytest.raises(native.LeoError):
        formats.decode_model(bytes(data))
    with pytest.raises(native.LeoError, match="duplicate"):
        formats.decode_model(_resign(data))


def test_overlapping_section_ranges_are_rejected():
    # lib.rs:1201-1208
    data = bytearray(formats.encode_model(_model()))
    second = HEADER + DESCRIPTOR
    data[second + 48:second + 56] = data[HEADER + 48:HEADER + 56]
    with pytest.raises(native.LeoError):
        formats.decode_model(bytes(data))
    with pytest.raises(native.LeoError, match="overlapping"):
        formats.decode_model(_resign(data))


def test_statistics_require_every_persisted_field():
    # lib.rs:1210-1214: a statistics section of eight fields is rejected
    data = bytearray(formats.encode_model(_model()))
    d = _descriptor(bytes(data), 10)
    struct.pack_into("<Q", data, d + 56, 64)
    with pytest.raises(native.LeoError, match="statistics length"):
        formats.decode_model(_resign(data))


def test_input_projection_requires_complete_weight_tensor():
    # lib.rs:1216-1223: an input section whose weight vector is cut short
    data = bytearray(formats.encode_model(_model()))
    d = _descriptor(bytes(data), 6)
    offset, length = struct.unpack_from("<QQ", data, d + 48)
    struct.pack_into("<Q", data, d + 56, length - 4)
    with pytest.raises(native.LeoError) as e:
        formats.decode_model(_resign(data))
    assert e.value.code == native.ERR_CORRUPT


def test_header_rules():
    good = formats.encode_model(_model())
    for mutate, code in ((lambda d: d.__setitem__(slice(0, 8), b"PSCLS099"), native.ERR_INCOMPATIBLE),
                         (lambda d: struct.pack_into("<I", d, 8, 2), native.ERR_INCOMPATIBLE),
                         (lambda d: struct.pack_into("<I", d, 12, 0x04030201), native.ERR_INCOMPATIBLE),
                         (lambda d: d.__setitem__(60, 1), native.ERR_CORRUPT),
                         (lambda d: struct.pack_into("<I", d, 28, 1), native.ERR_CORRUPT)):
        data = bytearray(good)
        mutate(data)
        with pytest.raises(native.LeoError) as e:
            formats.decode_model(_resign(data) if code == native.ERR_CORRUPT else bytes(data))
        assert e.value.code == code
    with pytest.raises(native.LeoError):
        formats.decode_model(good[:100])
    # the semantics contract must be the current one (lib.rs:551-558)
    data = bytearray(good)
    d = _descriptor(good, 12)
    offset = struct.unpack_from("<Q", data, d + 48)[0]
    struct.pack_into("<I", data, offset + 16, 2)  # another CUDA ABI version
    with pytest.raises(native.LeoError) as e:
        formats.decode_model(_resign(data))
    assert e.value.code == native.ERR_INCOMPATIBLE


def test_checkpoint_layout_follows_the_reference_field_table():
    model = _model()
    model.generation = 5
    model.parameter_revision = 9
    data = formats.encode_model(model)
    magic, version, endian, generation, count, flags, cfg_off, cfg_len = struct.unpack_from("<8sIIQIIQQ", data, 0)
    assert (magic, version, endian, generation, count, flags) == (b"PSCLS100", 1, 0x01020304, 5, 12, 0)
    assert data[48:96] == bytes(48)
    assert data[96:128] == _sha(data[:96] + bytes(32))
    n, s, f = 128, 8, 8
    cfg = toml_test_config()
    slots, e = cfg.context.max_order * cfg.context.slots_per_order, cfg.context.embedding_dim
    shapes = {1: (0, 0, 0, 0), 2: (n, 0, 0, 0), 3: (n, s, 0, 0), 4: (n, s, 0, 0), 5: (n * s, 0, 0, 0),
              6: (258, f, 0, 0), 7: (257, n, 0, 0), 8: (257, 0, 0, 0), 9: (slots, e, 257, 0), 10: (9, 0, 0, 0),
              11: (2, 0, 0, 0), 12: (5, 0, 0, 0)}
    dtypes = {5: 2, 7: 2, 8: 2, 11: 4, 12: 3}
    cursor = (HEADER + 12 * DESCRIPTOR + ALIGN - 1) // ALIGN * ALIGN
    payload = {}
    for i in range(12):
        d = HEADER + i * DESCRIPTOR
        kind, schema, dtype, rank = struct.unpack_from("<IIII", data, d)
        shape = struct.unpack_from("<4Q", data, d + 16)
        offset, length, alignment, compression = struct.unpack_from("<QQII", data, d + 48)
        assert kind == i + 1 and schema == 1 and dtype == dtypes.get(kind, 1)
        assert shape == shapes[kind] and rank == sum(1 for x in shape if x)
        assert offset == cursor and alignment == 64 and compression == 0
        assert data[d + 72:d + 104] == _sha(data[offset:offset + length]) and data[d + 104:d + 128] == bytes(24)
        payload[kind] = data[offset:offset + length]
        cursor = (offset + length + ALIGN - 1) // ALIGN * ALIGN
    assert len(data) == cursor
    assert (cfg_off, cfg_len) == struct.unpack_from("<QQ", data, HEADER + 48)
    assert payload[1].decode() == model.config.to_toml()
    assert struct.unpack("<QQ", payload[11]) == (5, 9)
    assert struct.unpack("<5I", payload[12]) == (1, 1, 1, 1, 1)
    assert struct.unpack_from("<Q", payload[8])[0] == 257
    assert np.array_equal(np.frombuffer(payload[8][8:], dtype="<f4"), model.bias)
    assert np.array_equal(np.frombuffer(payload[7][8:], dtype="<f4"), model.out_weight)
    t = payload[2]  # threshold, excitability, neuron types: length-prefixed
    assert struct.unpack_from("<Q", t)[0] == n
    assert np.array_equal(np.frombuffer(t[8:8 + 4 * n], dtype="<f4"), model.threshold)
    assert struct.unpack_from("<Q", payload[3])[0] == s  # capacity_per_neuron first
    st = struct.unpack("<QQdQQQQQQ", payload[10])
    assert st[0] == model.statistics["processed_bytes"] and len(payload[10]) == 72


def test_trained_model_round_trip(tmp_path, oracle):
    from tests.helpers import story

    model = _model()
    rt = oracle.OracleRuntime(model)
    rt.train_story_batch([story(5, 60), story(6, 50)], oracle.TRAINING, replay=True)
    trained = rt.model()
    assert trained.parameter_revision > 0 and trained.statistics["processed_bytes"] > 0
    path = tmp_path / "trained.pscls"
    formats.save_model_atomic(path, trained, False)
    loaded = formats.load_model(path)
    assert _equal(loaded, trained)
    # checkpoint.rs:64-79: runtime state is not part of a checkpoint
    resumed = oracle.OracleRuntime(loaded)
    assert len(resumed.read_list("active")) == 0


# --- LEODATA1 ----------------------------------------------------------------------
def _python_index(bytes_path, entries, provenance: bytes) -> bytes:
    """The LEODATA1 index in the layout of python/prepare_tinystories.py:200-262
    and lib.rs:237-323, written with struct and hashlib."""
    raw = open(bytes_path, "rb").read()
    records = b"".join(struct.pack("<QII", o, n, fl) for o, n, fl in entries)
    bytes_digest, records_digest = _sha(raw), _sha(records)
    h = hashlib.sha256(b"LEO-DATASET-ID\0")
    h.update(struct.pack("<IQQ", 1, len(entries), len(raw)))
    h.update(bytes_digest + records_digest + provenance)
    header = bytearray(192)
    header[0:8] = b"LEODATA1"
    struct.pack_into("<IIQQ", header, 8, 1, 192, len(entries), len(raw))
    header[32:64], header[64:96], header[96:128], header[128:160] = bytes_digest, records_digest, provenance, \
        h.digest()
    header[160:192] = _sha(bytes(header))
    return bytes(header) + records


def test_reads_story_by_offset_and_verifies_identity(tmp_path):
    # lib.rs:336-370
    b, idx = tmp_path / "d.bytes", tmp_path / "d.idx"
    b.write_bytes(b"onetwo")
    provenance = _sha(b"test provenance")
    identity = formats.write_index(idx, b, [formats.StoryIndex(0, 3), formats.StoryIndex(3, 3)], provenance)
    with formats.PreparedDataset.open(b, idx) as ds:
        assert ds.identity() == identity
        assert ds.story(1) == b"two" and ds.story(0) == b"one"
        assert len(ds) == 2 and ds.entry(1) == formats.StoryIndex(3, 3, 0) and ds.entry(2) is None
        data, offsets = ds.pack(0, 2)
        assert data.tobytes() == b"onetwo" and offsets.tolist() == [0, 3, 6]
    assert identity.dataset_id == formats.compute_dataset_id(1, 2, 6, _sha(b"onetwo"), identity.records_digest,
                                                             provenance)
    assert idx.read_bytes() == _python_index(b, [(0, 3, 0), (3, 3, 0)], provenance)


def test_changed_middle_bytes_are_rejected(tmp_path):
    # lib.rs:372-398
    b, idx = tmp_path / "m.bytes", tmp_path / "m.idx"
    b.write_bytes(b"abcdef")
    formats.write_index(idx, b, [formats.StoryIndex(0, 6)], bytes(32))
    b.write_bytes(b"abcXef")
    with pytest.raises(native.LeoError) as e:
        formats.PreparedDataset.open(b, idx)
    assert e.value.code == native.ERR_CORRUPT


def test_python_written_index_opens_and_rejections(tmp_path):
    rng = np.random.default_rng(11)
    stories = [("story %d " % i + "x" * int(rng.integers(1, 40)) + " é\n").encode() for i in range(30)]
    b = tmp_path / "p.bytes"
    b.write_bytes(b"".join(stories))
    entries, at = [], 0
    for s in stories:
        entries.append((at, len(s), int(rng.integers(0, 2))))
        at += len(s)
    provenance = _sha(b'{"split":"train"}')
    idx = tmp_path / "p.idx"
    idx.write_bytes(_python_index(b, entries, provenance))
    with formats.PreparedDataset.open(b, idx) as ds:
        assert [ds.story(i) for i in range(len(ds))] == stories
        assert ds.stories(3, 4) == stories[3:7]
        ident = ds.identity()
        assert (ident.record_count, ident.bytes_length, ident.provenance_digest) == (30, at, provenance)

    def rejected(mutate_index=None, entries_=None, bytes_=None):
        path_b, path_i = tmp_path / "r.bytes", tmp_path / "r.idx"
        path_b.write_bytes(bytes_ if bytes_ is not None else b.read_bytes())
        raw = bytearray(_python_index(path_b, entries_ or entries, provenance))
        if mutate_index:
            mutate_index(raw)
        path_i.write_bytes(bytes(raw))
        with pytest.raises(native.LeoError) as e:
            formats.PreparedDataset.open(path_b, path_i)
        return e.value

    assert "header SHA-256" in str(rejected(lambda r: r.__setitem__(20, r[20] ^ 1)))
    assert "magic" in str(rejected(lambda r: r.__setitem__(0, ord("X"))))
    assert "zero length" in str(rejected(entries_=entries[:3] + [(entries[3][0], 0, 0)]))
    assert "overlaps" in str(rejected(entries_=[(0, 5, 0), (4, 5, 0)]))
    assert "past the bytes file" in str(rejected(entries_=[(0, at + 1, 0)]))

    def bad_id(r):  # a wrong dataset ID under a valid header digest
        r[128] ^= 1
        r[160:192] = bytes(32)
        r[160:192] = _sha(bytes(r[:192]))

    assert "dataset ID" in str(rejected(bad_id))
    # a story that is not UTF-8 opens (the index is valid) but cannot be read
    path_b, path_i = tmp_path / "u.bytes", tmp_path / "u.idx"
    path_b.write_bytes(b"ok\xc3\x28")
    formats.write_index(path_i, path_b, [formats.StoryIndex(0, 2), formats.StoryIndex(2, 2)], bytes(32))
    with formats.PreparedDataset.open(path_b, path_i) as ds:
        assert ds.story(0) == b"ok"
        with pytest.raises(native.LeoError, match="UTF-8"):
            ds.story(1)


def test_write_index_rejects_invalid_ranges(tmp_path):
    b = tmp_path / "w.bytes"
    b.write_bytes(b"abc")
    with pytest.raises(native.LeoError):
        formats.write_index(tmp_path / "w.idx", b, [formats.StoryIndex(0, 4)], bytes(32))
    with pytest.raises(native.LeoError):
        formats.write_index(tmp_path / "w.idx", b, [formats.StoryIndex(1, 2), formats.StoryIndex(0, 1)], bytes(32))
