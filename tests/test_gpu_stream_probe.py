"""The bench's stream probes (velograd_amd/csrc/stream_probe.hip) move every byte they are timed
for: a shape that skipped part of its buffers would read as faster than the hardware allows.
Each byte pattern is run on small buffers (a whole number of tiles plus a ragged tail) and its
outputs checked element by element: written streams hold the sum of the read streams (as 32-bit
lanes), the second write stream that sum with every lane's lowest bit flipped, placed by the
rotation rule; read-only shapes write nothing; write-only shapes write their unit index."""

import ctypes

import numpy as np
import pytest
import torch

from velograd_amd.build import PROBE_LIB_PATH

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _lib():
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    lib.velograd_stream_probe_shape.restype = ctypes.c_int32
    lib.velograd_stream_probe_shape.argtypes = (
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        + [ctypes.c_int32] * 5 + [ctypes.c_void_p])
    lib.velograd_stream_probe.restype = ctypes.c_int32
    lib.velograd_stream_probe.argtypes = ([ctypes.c_int32] + [ctypes.c_void_p] * 4
                                          + [ctypes.c_int64, ctypes.c_void_p])
    return lib


def _expected_second_write(s, n16, tile, vpt, lane_units, rotate):
    """Where the second write stream's value for unit i lands: in whole tiles, the vector of slot
    k goes to slot (k + vpt / 2) % vpt of the same tile; elsewhere to i itself."""
    out = np.empty_like(s)
    for i in range(n16):
        t = i // tile
        if rotate and vpt >= 2 and (t + 1) * tile <= n16:
            within = i - t * tile
            block_units = tile // vpt             # block * lane_units
            k, rest = divmod(within, block_units)
            j = t * tile + ((k + vpt // 2) % vpt) * block_units + rest
        else:
            j = i
        out[j] = s[i] ^ 1
    return out


SHAPES = [
    # (nread, nwrite, block, vpt, lane_bytes, wgs_per_cu, flags)
    (2, 2, 256, 2, 16, 0, 7), (2, 2, 256, 2, 16, 0, 7 | 8), (2, 2, 256, 2, 16, 0, 3),
    (2, 2, 512, 4, 32, 0, 7), (2, 2, 1024, 1, 16, 2, 7 | 8), (2, 2, 256, 2, 16, 0, 4),
    (2, 1, 512, 1, 16, 0, 7), (2, 1, 256, 4, 16, 0, 7 | 8), (2, 1, 256, 2, 16, 1, 7),
    (3, 1, 1024, 1, 16, 0, 7), (3, 1, 256, 2, 32, 4, 7 | 8),
    (1, 1, 512, 1, 16, 0, 7), (1, 1, 256, 2, 16, 0, 2),
    (2, 0, 256, 2, 16, 0, 7), (2, 0, 512, 1, 16, 2, 7),
    (0, 2, 256, 2, 16, 0, 7), (0, 2, 256, 4, 32, 0, 7 | 8),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[
    f"{s[0]}R{s[1]}W-b{s[2]}-v{s[3]}-l{s[4]}-p{s[5]}-f{s[6]}" for s in SHAPES])
def test_probe_shape_moves_every_byte(shape):
    nr, nw, block, vpt, lane, wpc, flags = shape
    lib = _lib()
    tile = vpt * block * (lane // 16)
    n16 = 5 * tile + tile // 2 + 3           # whole tiles and a ragged tail
    print(f"stream probe shape {shape}, n16 {n16}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(sum(shape))
    rd = [torch.randint(0, 2 ** 31, (n16, 4), device=DEV, dtype=torch.int64, generator=g)
          .to(torch.int32) for _ in range(3)]
    sentinel = -123456789
    wr = [torch.full((n16, 4), sentinel, device=DEV, dtype=torch.int32) for _ in range(2)]
    rdp = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in rd])
    wrp = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in wr])
    rc = lib.velograd_stream_probe_shape(nr, nw, ctypes.cast(rdp, ctypes.c_void_p),
                                         ctypes.cast(wrp, ctypes.c_void_p), n16, block, vpt,
                                         lane, wpc, flags, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    a = [t.cpu().numpy().astype(np.uint32) for t in rd]
    w = [t.cpu().numpy().astype(np.uint32) for t in wr]
    if nr == 0:
        s = np.zeros((n16, 4), np.uint32)
        s[:, 0] = np.arange(n16, dtype=np.uint32)
        s[:, 1], s[:, 2], s[:, 3] = 1, 2, 3
    else:
        s = sum(a[:nr]).astype(np.uint32)
    untouched = np.full((n16, 4), sentinel, np.int32).astype(np.uint32)
    if nw == 0:
        assert np.array_equal(w[0], untouched) and np.array_equal(w[1], untouched)
        return
    assert np.array_equal(w[0], s), "first write stream"
    if nw == 2:
        want = _expected_second_write(s, n16, tile, vpt, lane // 16, (flags & 4) != 0)
        assert np.array_equal(w[1], want), "second write stream"
    else:
        assert np.array_equal(w[1], untouched)


@pytest.mark.parametrize("pattern,nr,nw", [(0, 1, 1), (1, 2, 2), (2, 2, 1), (3, 2, 0), (4, 0, 2),
                                           (5, 3, 1)])
def test_bench_ceiling_patterns_move_every_byte(pattern, nr, nw):
    """velograd_stream_probe's fixed shapes (256 threads, two 16-byte vectors, second write
    stream rotated): a, b read; c, d written; pattern 5 reads a, b, d and writes c."""
    lib = _lib()
    tile = 512
    n16 = 7 * tile + 100
    print(f"bench ceiling pattern {pattern}, n16 {n16}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(pattern)
    bufs = [torch.randint(0, 2 ** 31, (n16, 4), device=DEV, dtype=torch.int64, generator=g)
            .to(torch.int32) for _ in range(4)]
    orig = [b.cpu().numpy().astype(np.uint32) for b in bufs]
    rc = lib.velograd_stream_probe(pattern, *[b.data_ptr() for b in bufs], n16,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    got = [b.cpu().numpy().astype(np.uint32) for b in bufs]
    if pattern == 5:
        s = (orig[0] + orig[1] + orig[3]).astype(np.uint32)
    elif nr == 0:
        s = np.zeros((n16, 4), np.uint32)
        s[:, 0] = np.arange(n16, dtype=np.uint32)
        s[:, 1], s[:, 2], s[:, 3] = 1, 2, 3
    else:
        s = sum(orig[:nr]).astype(np.uint32)
    if nw == 0:
        assert np.array_equal(got[2], orig[2]) and np.array_equal(got[3], orig[3])
        return
    assert np.array_equal(got[2], s)
    if nw == 2:
        assert np.array_equal(got[3], _expected_second_write(s, n16, tile, 2, 1, True))
    elif pattern != 5:
        assert np.array_equal(got[3], orig[3])
