"""The committed fixtures (tests/golden/qmm_golden.npz, written by make_golden.py).

CPU: both oracle restatements reproduce every stored dequant bit for bit and every stored
fp64 result, and the known-answer unpack words decode as stored.  GPU: the fast kernel and
the generic path meet the 1e-2 bar on every fixture.
"""
import os

import numpy as np
import pytest

from oracle import qmm_oracle as Q

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qmm_golden.npz")


def load_cases():
    z = np.load(PATH, allow_pickle=False)
    cases = []
    for name in z["cases"]:
        name = str(name)
        M, N, K, bits, gs, dt, lb = (int(v) for v in z[f"{name}/meta"])
        c = Q.QmmCase(x=z[f"{name}/x"], w=z[f"{name}/w"], scales=z[f"{name}/scales"],
                      biases=z[f"{name}/biases"], M=M, N=N, K=K, bits=bits, gs=gs, xdt=dt,
                      sdt=dt, lbias=z[f"{name}/lbias"] if lb else None)
        cases.append((name, c, z[f"{name}/dequant"], z[f"{name}/y_f64"]))
    return z, cases


def test_known_answer_words(oracle):
    z, _ = load_cases()
    assert np.array_equal(Q.unpack(z["known_w4"], 4, 16), z["known_codes4"])
    assert np.array_equal(oracle.unpack(z["known_w8"], 8, 1, 8), z["known_codes8"])


def test_oracle_reproduces_fixtures(oracle):
    _, cases = load_cases()
    assert len(cases) >= 7
    for name, c, dq, y in cases:
        got = oracle.dequant(c.w, c.scales, c.biases, c.sdt, c.bits, c.gs, c.N, c.K)
        assert np.array_equal(got.view(np.uint32), dq.view(np.uint32)), name
        assert np.array_equal(Q.dequant(c.w, c.scales, c.biases, c.sdt, c.bits, c.gs, c.K)
                              .view(np.uint32), dq.view(np.uint32)), name
        assert np.allclose(oracle.qmm_f64(c), y, rtol=1e-13, atol=1e-13), name


@pytest.mark.gpu
def test_gpu_paths_match_fixtures(ctx):
    from gpu_util import announce, download, upload
    _, cases = load_cases()
    for name, c, _, y in cases:
        x, w, s, b, lb = upload(c)
        announce(f"golden {name}")
        if ctx.supported(c.M, c.N, c.K, c.bits, c.gs, c.xdt):
            rel, ok = Q.tolerance_check(download(ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)), y)
            assert rel <= 1e-2 and ok, (name, rel)
        rel, ok = Q.tolerance_check(download(ctx.fallback(x, w, s, b, c.bits, c.gs, lbias=lb)), y)
        assert rel <= 1e-2 and ok, (name, "generic", rel)
