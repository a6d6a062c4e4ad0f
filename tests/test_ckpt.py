"""ckpt.rs format (rustnn_amd/ckpt.py), host side.

The reference's own checkpoint tests (ckpt.rs:299-368) restated over a fake
model of two parameters and a buffer: round trip with the magic, a different
configuration refused, a truncated file refused, a legacy headerless file
accepted, a failed save leaving the previous file and no .tmp.  FNV-1a 64 is
pinned to its published test vectors; the header bytes are checked field by
field."""
import os
import struct

import numpy as np
import pytest

from rustnn_amd import ckpt


def fake(fill):
    """Fake::new (ckpt.rs:263-277): params of 6 and 4 values, a buffer of 3."""
    p0 = np.array([fill + j for j in range(6)], np.float32)
    p1 = np.array([fill + 10.0 + j for j in range(4)], np.float32)
    return [p0, p1, np.full(3, fill * 2.0, np.float32)]


LENS = [6, 4, 3]


def test_fnv1a_published_vectors():
    assert ckpt.config_hash(b"", []) == 0xCBF29CE484222325
    assert ckpt.config_hash(b"a", []) == 0xAF63DC4C8601EC8C
    assert ckpt.config_hash(b"foobar", []) == 0x85944171F73967E8
    # u64 fields are hashed as their 8 little-endian bytes
    assert ckpt.config_hash(b"x", [0x0102]) == ckpt.config_hash(b"x\x02\x01" + b"\0" * 6, [])


def test_round_trip_and_header(tmp_path):
    path = str(tmp_path / "roundtrip.bin")
    saved = fake(1.5)
    ckpt.save(path, saved, 0xABCD)
    loaded = ckpt.load(path, LENS, 0xABCD)
    for a, b in zip(saved, loaded):
        assert np.array_equal(a, b)
    data = open(path, "rb").read()
    assert data.startswith(b"RUSTNN\0")
    assert struct.unpack_from("<IQQ", data, 7) == (3, 13, 0xABCD)
    assert len(data) == ckpt.HEADER_LEN + 13 * 4
    assert not os.path.exists(path + ".tmp")


def test_refuses_other_configuration(tmp_path):
    path = str(tmp_path / "config.bin")
    ckpt.save(path, fake(1.0), 0x1111)
    with pytest.raises(ckpt.CheckpointError, match="another configuration"):
        ckpt.load(path, LENS, 0x2222)
    with pytest.raises(ckpt.CheckpointError, match="tensors"):
        ckpt.load(path, [6, 4, 2, 1], 0x1111)


def test_refuses_truncated(tmp_path):
    path = str(tmp_path / "trunc.bin")
    ckpt.save(path, fake(1.0), 7)
    data = open(path, "rb").read()
    open(path, "wb").write(data[:-8])
    with pytest.raises(ckpt.CheckpointError):
        ckpt.load(path, LENS, 7)
    open(path, "wb").write(data[:10])
    with pytest.raises(ckpt.CheckpointError):
        ckpt.load(path, LENS, 7)


def test_accepts_legacy_headerless(tmp_path, capsys):
    path = str(tmp_path / "legacy.bin")
    original = fake(3.0)
    ckpt.save(path, original, 42)
    data = open(path, "rb").read()
    open(path, "wb").write(data[ckpt.HEADER_LEN:])
    loaded = ckpt.load(path, LENS, 42)
    assert np.array_equal(loaded[0], original[0]) and np.array_equal(loaded[2], original[2])
    assert "legacy" in capsys.readouterr().err


def test_failed_save_keeps_previous(tmp_path):
    path = str(tmp_path / "atomic.bin")
    ckpt.save(path, fake(5.0), 1)
    good = open(path, "rb").read()
    bad = os.path.join(path, "not-a-directory")
    with pytest.raises(OSError):
        ckpt.save(bad, fake(9.0), 1)
    assert open(path, "rb").read() == good
    assert not os.path.exists(bad + ".tmp")


def test_resnet_buffer_layout():
    """ResNet-20's BN buffers: stem + 9 blocks x 2 + 2 shortcuts = 21 BNs."""
    class N:
        depth_n, width = 3, 32
    lens = ckpt._resnet_buffer_lens(N)
    assert len(lens) == 42 and sum(lens) == 2 * (32 + 6 * 32 + 6 * 64 + 6 * 128 + 64 + 128)


def test_fnv1a_entry_points():
    """rnn_fnv1a_bytes / rnn_fnv1a_f32 (host functions of librnn.so): the
    published FNV-1a 64 vectors, and a float hashed as its 4 little-endian
    bytes."""
    import ctypes as C
    from rustnn_amd import lib
    L = lib()
    off = 0xCBF29CE484222325
    for s, want in ((b"", 0xCBF29CE484222325), (b"a", 0xAF63DC4C8601EC8C),
                    (b"foobar", 0x85944171F73967E8)):
        assert L.rnn_fnv1a_bytes(C.c_uint64(off), C.c_char_p(s), len(s)) == want
    v = np.array([1.5, -0.0, np.float32(3.1415927)], np.float32)
    got = L.rnn_fnv1a_f32(C.c_uint64(off), v.ctypes.data, 3)
    raw = v.tobytes()  # little-endian on this host
    assert got == L.rnn_fnv1a_bytes(C.c_uint64(off), C.c_char_p(raw), len(raw))
