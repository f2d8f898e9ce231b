"""The TMAC weight-file loader (tmac_model_load; reference load_tmac,
tmac_gguf.cpp:1372-1425).  Files are written here exactly as the reference's
writer does (scripts/extract_tmac.py:261-272, 317-327: b"TMAC", u64 count,
then u64 name_len, name, u64 rows, u64 cols, u32 type, u64 n_bytes, data), and
the loaded table and bytes must round-trip.  CPU tests load into host memory
(no context); the GPU test loads onto the device and runs a projection on a
loaded tensor."""
import ctypes
import struct

import numpy as np
import pytest

import oracle
import tmac_attn


def write_tmac(path, tensors, magic=b"TMAC", count=None):
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<Q", len(tensors) if count is None else count))
        for name, rows, cols, ttype, data in tensors:
            nb = name.encode() if isinstance(name, str) else name
            f.write(struct.pack("<Q", len(nb)))
            f.write(nb)
            f.write(struct.pack("<Q", rows))
            f.write(struct.pack("<Q", cols))
            f.write(struct.pack("<I", ttype))
            f.write(struct.pack("<Q", len(data)))
            f.write(data)


def sample_tensors(rng):
    long_name = "blk.0." + "x" * 200
    return [
        ("token_embd.weight", 16, 64, 8, rng.integers(0, 256, 16 * 2 * 34, dtype=np.uint8).tobytes()),
        ("blk.0.attn_q.weight", 32, 64, 6, rng.integers(0, 256, 32 * 2 * 22, dtype=np.uint8).tobytes()),
        ("blk.0.attn_q.bias", 32, 1, 0, rng.standard_normal(32).astype(np.float32).tobytes()),
        (long_name, 3, 1, 0, b"\x01" * 12),
        ("blk.0.attn_q.weight", 1, 1, 0, b"\x00" * 4),  # a duplicate name: lookups see the first
        ("empty", 0, 0, 0, b""),
        ("blk.0.ffn_down.weight", 2, 256, 14, rng.integers(0, 256, 2 * 210, dtype=np.uint8).tobytes()),
    ]


def test_load_round_trip_host(tmp_path):
    rng = np.random.default_rng(1)
    ts = sample_tensors(rng)
    path = tmp_path / "m.tmac"
    write_tmac(path, ts)
    m = tmac_attn.Model(str(path))
    try:
        assert len(m) == len(ts)
        for i, (name, rows, cols, ttype, data) in enumerate(ts):
            t = m.tensor(i)
            assert t["name"] == name[:127]
            assert (t["rows"], t["cols"], t["type"], t["n_bytes"]) == (rows, cols, ttype, len(data))
            if data:
                assert ctypes.string_at(t["data"], len(data)) == data
                assert t["data"] % 256 == 0
        first = m.find("blk.0.attn_q.weight")
        assert first["rows"] == 32 and first["type"] == 6
        assert m.find("blk.0." + "x" * 121)["n_bytes"] == 12  # cut to 127 characters
        assert m.find("missing") is None
    finally:
        m.free()


@pytest.mark.parametrize("mutate", ["magic", "truncated_data", "truncated_header", "count"])
def test_rejects_bad_files(tmp_path, mutate):
    rng = np.random.default_rng(2)
    path = tmp_path / "bad.tmac"
    ts = sample_tensors(rng)
    if mutate == "magic":
        write_tmac(path, ts, magic=b"GGUF")
    elif mutate == "count":
        write_tmac(path, ts, count=10 ** 9)
    else:
        write_tmac(path, ts)
        raw = path.read_bytes()
        cut = len(raw) - 100 if mutate == "truncated_data" else 40
        path.write_bytes(raw[:cut])
    with pytest.raises(tmac_attn.TmacError) as e:
        tmac_attn.Model(str(path))
    assert e.value.status == tmac_attn.TMAC_ERR_IO


def test_missing_file(tmp_path):
    with pytest.raises(tmac_attn.TmacError) as e:
        tmac_attn.Model(str(tmp_path / "nope.tmac"))
    assert e.value.status == tmac_attn.TMAC_ERR_IO


@pytest.mark.gpu
def test_device_load_and_project(ctx, tmp_path):
    """Load onto the device, read a tensor back, and run the Q5_0 projection on it."""
    rng = np.random.default_rng(3)
    ts = sample_tensors(rng)
    path = tmp_path / "m.tmac"
    write_tmac(path, ts)
    m = tmac_attn.Model(str(path), ctx)
    try:
        t = m.find("blk.0.attn_q.weight")
        host = np.empty(t["n_bytes"], np.uint8)
        ctx._check(ctx.lib.tmac_memcpy_d2h(ctx.handle, None, host.ctypes.data, t["data"], t["n_bytes"]), "d2h")
        ctx.synchronize()
        assert host.tobytes() == ts[1][4]
        # scales sane for a numeric check: rewrite the fp16 d of every block on the device copy
        blocks = host.reshape(-1, 22).copy()
        blocks[:, 0:2] = np.full(blocks.shape[0], 0.01, np.float16).view(np.uint8).reshape(-1, 2)
        ctx._check(ctx.lib.tmac_memcpy_h2d(ctx.handle, None, t["data"], blocks.ctypes.data, blocks.size), "h2d")
        ctx.synchronize()
        x = rng.standard_normal(64).astype(np.float32)
        dx, dy = ctx.upload(x), ctx.empty(32)
        ctx.matmul(tmac_attn.TMAC_Q5_0, 32, 64, t["data"], dx, dy)
        ref = oracle.matmul_q(oracle.Q5_0, blocks.reshape(-1), x, 32, 64)
        np.testing.assert_allclose(dy.numpy(), ref, rtol=1e-4, atol=2e-5)
    finally:
        m.free()
