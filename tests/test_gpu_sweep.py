"""A seeded sweep of random shapes through the fast kernel (the C ABI), each against the CPU
oracle and bit-identical on a repeat call.

The fixed cases of test_gpu_parity.py pin each split the planner has; this sweep draws rows,
N, K, format and dtype at random (seed fixed), so that the planner's rules meet shapes nobody
picked: ragged N, K of any whole number of super-steps, 1..16 rows, with and without a
linear bias.  Sizes stay where the fp64 oracle takes at most a second or two.
"""
import numpy as np
import pytest

from gpu_util import announce, download, upload
from oracle.qmm_oracle import BF16, F16, make_case, tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2


def kss(bits, gs):
    """k of one super-step (the kernels' smallest K step)."""
    return (512 // bits) * ((2 if gs == 128 else 1) if bits == 4 else gs // 32)


def sweep_cases(n, seed, nk_min, nk_max, n_max, k_max, m_min=1, k_min=1, whole_chunks=False):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        bits = int(rng.choice([4, 8]))
        gs = int(rng.choice([32, 64, 128]))
        M = int(rng.integers(m_min, 17))
        # whole_chunks: K a multiple of 8 groups, which 9..16 rows take in one launch
        step = 8 * gs if whole_chunks else kss(bits, gs)
        K = step * int(rng.integers(max(1, -(-k_min // step)), max(2, k_max // step)))
        N = int(rng.integers(1, n_max))
        if not nk_min <= N * K <= nk_max:
            continue
        dt = BF16 if rng.random() < 0.6 else F16
        lb = bool(rng.random() < 0.3)
        cases.append((M, N, K, bits, gs, dt, lb))
    return cases


# 100 small shapes, 20 of 12..48 M weights (long K and wide N: several k-blocks, the tree
# of exchanges, the second pass, one k-block at 9..12 rows), and 20 at 9..16 rows with
# K >= 12288 (two k-blocks of up to 24 whole tiles, trees of four to eight k-blocks)
CASES = (sweep_cases(100, 20261202, 1, 12_000_000, 6000, 12288)
         + sweep_cases(20, 1202, 12_000_001, 48_000_000, 40000, 32768)
         + sweep_cases(20, 31202, 24_000_000, 160_000_000, 16000, 32768, m_min=9, k_min=12288,
                       whole_chunks=True))


@pytest.mark.parametrize("M,N,K,bits,gs,dt,lb", CASES)
def test_random_shape_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs, dt, lb):
    import torch
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=M * 7919 + N * 31 + K + bits + gs,
                  lbias=lb)
    try:  # 9..16 rows with one-super-step chunks run as two launches of up to 8 rows
        p = ctx.plan(M, N, K, bits, gs)
        split = f"nkb={p['nkb']} Gkb={p['Gkb']} aligned={p['aligned']} reduce={p['reduce']}"
    except RuntimeError:
        split = "two launches of up to 8 rows"
    announce(f"sweep M={M} N={N} K={K} bits={bits} gs={gs} dt={dt} lbias={lb} {split}")
    x, w, s, b, lbd = upload(c)
    y = ctx.qmm(x, w, s, b, bits, gs, lbias=lbd)
    torch.cuda.synchronize()
    rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"
    y2 = ctx.qmm(x, w, s, b, bits, gs, lbias=lbd)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
