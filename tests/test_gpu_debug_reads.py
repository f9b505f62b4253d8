"""The two bandwidth references the bench reports, checked for reading exactly what they
claim: each wave's word in the sink is lane 0's XOR of every 16-byte word it loaded, which
is recomputed here on the CPU from the split.

- dfq_read_stream: wave g of the grid reads 4 KB blocks g, g + 8G, ...; lane 0 the first 16
  bytes of each kilobyte.
- dfq_debug_read_units: the fast kernel's own loads for a 4-bit g64 shape; wave w of a
  workgroup reads units a + w, a + w + 12, ... of the workgroup's range [a, b); lane 0 (row
  0 of the unit's tile, lane group 0) loads the scales of its row for the unit's 8 groups and
  four 16-byte weight pieces, 64 bytes apart, from the start of the unit's 256 bytes.
"""
import numpy as np
import pytest

from gpu_util import announce

pytestmark = pytest.mark.gpu


def _xor_words(words16: np.ndarray) -> int:
    """XOR of 16-byte words (rows of 4 uint32), folded to one uint32."""
    if words16.size == 0:
        return 0
    v = np.bitwise_xor.reduce(words16, axis=0)
    return int(v[0] ^ v[1] ^ v[2] ^ v[3])


def test_read_stream_reads_its_blocks(ctx):
    import torch
    G = ctx.num_cus
    units = 8 * G * 3 + 37                       # not a multiple of the waves
    rng = np.random.default_rng(5)
    src = rng.integers(0, 2**32, size=(units * 256, 4), dtype=np.uint32)
    d = torch.from_numpy(src.view(np.int32)).cuda()
    sink = torch.zeros(8 * G, dtype=torch.int32, device="cuda")
    announce(f"read_stream units={units}")
    ctx.read_stream(d, units * 4096, sink)
    torch.cuda.synchronize()
    got = sink.cpu().numpy().view(np.uint32)
    nw = 8 * G
    for g in range(nw):
        blocks = np.arange(g, units, nw)
        idx = (blocks[:, None] * 256 + np.arange(4)[None, :] * 64).reshape(-1)
        assert got[g] == _xor_words(src[idx]), g


@pytest.mark.parametrize("M,N,K", [(8, 17408, 5120), (1, 5000, 4096)])
def test_read_units_reads_the_kernels_units(ctx, M, N, K):
    import torch
    p = ctx.plan(M, N, K, 4, 64)
    assert p["nkb"] == 1 and p["ch"] == 4
    rng = np.random.default_rng(M + N)
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint32)
    s = rng.integers(0, 2**16, size=(N, K // 64), dtype=np.uint16)
    b = rng.integers(0, 2**16, size=(N, K // 64), dtype=np.uint16)
    wd = torch.from_numpy(w.view(np.int32)).cuda()
    sd = torch.from_numpy(s.view(np.int16)).cuda().view(torch.bfloat16)
    bd = torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16)
    sink = torch.zeros(12 * ctx.num_cus, dtype=torch.int32, device="cuda")
    announce(f"read_units M={M} N={N} K={K} plan={p}")
    ctx.read_units(wd, sd, bd, M, N, K, sink)
    torch.cuda.synchronize()
    got = sink.cpu().numpy().view(np.uint32)
    SS, T, G = p["SS"], p["T"], p["Gkb"]
    U = T * SS
    base, rem = U // G, U % G
    wbytes = w.view(np.uint8).reshape(N, K // 2)
    sbytes = s.view(np.uint8).reshape(N, K // 32)
    for wg in range(G):
        a = wg * base + min(wg, rem)
        e = a + base + (1 if wg < rem else 0)
        for wave in range(12):
            words = []
            for u in range(a + wave, e, 12):
                t, c = divmod(u, SS)
                row = t * 16
                words.append(np.frombuffer(sbytes[row, c * 16:c * 16 + 16].tobytes(), np.uint32))
                for j in range(4):
                    o = c * 256 + j * 64
                    words.append(np.frombuffer(wbytes[row, o:o + 16].tobytes(), np.uint32))
            want = _xor_words(np.array(words).reshape(-1, 4)) if words else 0
            assert got[wg * 12 + wave] == want, (wg, wave)
