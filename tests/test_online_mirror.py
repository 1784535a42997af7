"""The streaming kernel's one-pass online softmax, mirrored in C++ on the CPU.

``oracle/online_mirror.cpp`` restates the recurrence of the row-per-wave
kernel (rescale folded into the accumulate, ``acc = acc*c + x`` on a new
maximum, ``acc += p*x`` otherwise).  It is built here with AddressSanitizer and
UndefinedBehaviorSanitizer and checked against the float64 two-pass softmax of
``attnres_oracle.route`` on random inputs and on logit orders that drive each
branch (rising: every source a new maximum; falling: none after the first;
equal), at the fp32 bar of the GPU parity tests:
``|out - ref| <= 1e-5 |ref| + 1e-6 max|ref|``, lse within ``1e-5 (1 + |lse|)``.
A planted mistake (the rescale dropped on a new maximum) must fail that bar.
"""

import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import attnres_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "online_mirror.cpp")


@pytest.fixture(scope="module")
def mirror(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("mirror") / "online_mirror")
    subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", SRC, "-o", exe], check=True)
    return exe


def run_mirror(exe, tmp_path, src, qw, eps):
    S, N, D = src.shape
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        f.write(np.array([S, N, D], dtype=np.int32).tobytes())
        f.write(np.array([eps], dtype=np.float32).tobytes())
        f.write(src.astype(np.float32).tobytes())
        f.write(qw.astype(np.float32).tobytes())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    subprocess.run([exe, str(fin), str(fout)], check=True, env=env)
    raw = np.fromfile(fout, dtype=np.float32)
    return raw[: N * D].reshape(N, D).astype(np.float64), raw[N * D:].astype(np.float64)


def close_f32(out, ref):
    tol = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max()
    return bool((np.abs(out - ref) <= tol).all())


def case(kind, S, N, D, seed):
    """bf16-exact sources and query; `kind` shapes the order of the logits."""
    rng = np.random.default_rng(seed)
    qw = O.bf16_round(rng.standard_normal(D) * 0.05)
    noise = rng.standard_normal((S, N, D))
    if kind == "random":
        src = noise * np.exp(rng.uniform(np.log(0.3), np.log(5.0), size=(S, 1, 1)))
    elif kind == "equal":
        src = np.broadcast_to(noise[:1], (S, N, D)).copy()
    else:
        # x_s = noise orthogonal to qw + b_s sqrt(D) qw/|qw|: logit_s = b_s sqrt(D) |qw| / sqrt(1 + b_s^2),
        # increasing in b_s; b spans logits of about -5 .. 5
        qh = qw / np.linalg.norm(qw)
        perp = noise - (noise @ qh)[..., None] * qh
        b = np.linspace(-0.1, 0.1, S) if kind == "rising" else np.linspace(0.1, -0.1, S)
        src = perp + b[:, None, None] * np.sqrt(D) * qh[None, None, :]
    return O.bf16_round(src), qw


CASES = [("random", s, 7, 512, 10 + s) for s in (1, 2, 3, 5, 8, 9, 16)] + [
    ("rising", 9, 5, 1024, 1),
    ("falling", 9, 5, 1024, 2),
    ("equal", 4, 3, 256, 3),
    ("random", 7, 3, 3072, 4),
]


@pytest.mark.parametrize("kind,S,N,D,seed", CASES, ids=[f"{c[0]}-S{c[1]}-D{c[3]}" for c in CASES])
def test_online_recurrence_matches_two_pass_softmax(mirror, tmp_path, kind, S, N, D, seed):
    src, qw = case(kind, S, N, D, seed)
    eps = 1e-5
    out, lse = run_mirror(mirror, tmp_path, src, qw, eps)
    ref = O.route(src, qw, eps)
    assert close_f32(out, ref["out"][0]), f"{kind} S={S}: worst err {np.abs(out - ref['out'][0]).max():.3e}"
    np.testing.assert_allclose(lse, ref["lse"][0], rtol=1e-5, atol=1e-5)
    if kind == "rising":  # the logits really are ordered as intended
        assert np.all(np.diff(ref["logits"][0], axis=1) > 0)
    if kind == "falling":
        assert np.all(np.diff(ref["logits"][0], axis=1) < 0)


def test_no_sources_is_nan(mirror, tmp_path):
    out, lse = run_mirror(mirror, tmp_path, np.zeros((0, 2, 64)), np.ones(64), 1e-5)
    assert np.isnan(out).all() and np.isnan(lse).all()


def test_dropped_rescale_fails_the_bar(tmp_path):
    # the recurrence without the rescale on a new maximum (acc = acc + x)
    # must not pass: rising logits make every source a new maximum
    src, qw = case("rising", 9, 5, 1024, 1)
    ref = O.route(src, qw, 1e-5)["out"][0]
    x = src.astype(np.float32)
    r = 1.0 / np.sqrt((x * x).mean(-1) + 1e-5)
    logit = (x @ qw.astype(np.float32)) * r  # (S, N)
    acc = np.zeros(x.shape[1:], dtype=np.float32)
    m = np.full(x.shape[1], -np.inf, dtype=np.float32)
    l = np.zeros(x.shape[1], dtype=np.float32)
    for s in range(x.shape[0]):
        new = logit[s] > m
        c = np.exp(np.where(new, m - logit[s], 0.0)).astype(np.float32)
        p = np.exp(np.where(new, 0.0, logit[s] - m)).astype(np.float32)
        l = np.where(new, l * c + 1, l + p)
        acc = np.where(new[:, None], acc + x[s], acc + p[:, None] * x[s])  # planted: no acc * c
        m = np.maximum(m, logit[s])
    assert not close_f32(acc / l[:, None], ref)
