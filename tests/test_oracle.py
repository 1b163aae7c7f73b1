"""Pins for the CPU oracle (oracle/lse_oracle.c, oracle/oracle.py) before it is
trusted as the parity checker.

Each pin is chosen so that a plausible slip in the restatement (a dropped LUT
term, a wrong index or shift, a mis-ordered tree level, a wrong identity or
alignment prefix) fails at least one check:

* the compiled reference (oracle/_ref, built from intlse/cpu/lse_kernel_simd.c)
  and the fixtures it wrote (tests/golden/) pin the Q16.16 pair op, the CPU
  quantisers and the whole AVX2 block tree bit for bit;
* closed forms and exhaustive error bounds pin the pair ops and tables;
* hand-computable special rows pin the GPU reduction tree shape;
* the reference's published accuracy envelopes (mean |err| vs fp64 per N,
  experiment_microbenchmark/*/outputs/*.json) pin the GPU trees statistically.
"""

import math
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")
NEG = O.GPU_NEG_INF


# ---------------------------------------------------------------------------
# compiled reference + golden fixtures
# ---------------------------------------------------------------------------
def _fixture_rows():
    d = np.load(os.path.join(GOLD, "intlse_cpu_ref.npz"))
    off = 0
    for (B, N) in d["shapes"]:
        n = int(B * N)
        yield d["x"][off:off + n].reshape(B, N), int(B)
        off += n


def test_intlse_cpu_restatement_matches_fixtures():
    d = np.load(os.path.join(GOLD, "intlse_cpu_ref.npz"))
    got, got_ni = [], []
    for x, _ in _fixture_rows():
        got.append(O.intlse_cpu_rows(x, False))
        got_ni.append(O.intlse_cpu_rows(x, True))
    np.testing.assert_array_equal(np.concatenate(got).view(np.int32), d["out"].view(np.int32))
    np.testing.assert_array_equal(np.concatenate(got_ni).view(np.int32), d["out_neg_inf"].view(np.int32))


def test_q16_pair_sweep_matches_fixture():
    """N=2 rows: scalar quantiser and one scalar pair over a dense gap sweep."""
    d = np.load(os.path.join(GOLD, "q16_pair_ref.npz"))
    np.testing.assert_array_equal(O.intlse_cpu_rows(d["x"]).view(np.int32), d["out"].view(np.int32))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("N", [2, 5, 63, 64, 65, 128, 191, 192, 640, 1000, 4096, 50257])
@pytest.mark.parametrize("rng_kind", ["u1", "u100", "u500", "wide"])
def test_intlse_cpu_restatement_matches_compiled_reference(N, rng_kind):
    rng = np.random.default_rng(N)
    lo, hi = {"u1": (-1, 0), "u100": (-100, 0), "u500": (-500, 0), "wide": (-2e4, 2e4)}[rng_kind]
    x = (rng.random((6, N)) * (hi - lo) + lo).astype(np.float32)
    x[1, ::5] = -np.inf
    if N > 3:
        x[2, 3] = np.float32(4e9)
        x[3, 0] = np.float32(-4e9)
    for ni in (False, True):
        np.testing.assert_array_equal(O.intlse_cpu_rows(x, ni).view(np.int32),
                                      O.ref_intlse_cpu_rows(x, ni).view(np.int32))


# ---------------------------------------------------------------------------
# Q16.16 pair op
# ---------------------------------------------------------------------------
def test_q16_pair_closed_forms():
    x = np.array([0, 12345, -987654, 2 ** 24], np.int32)
    # pair(x, x) = x + 1.0 (log2 2 = 1): M = 65536, LUT[(65536>>10)&63] = LUT[0] = 0
    np.testing.assert_array_equal(O.q16_pair(x, x), x + 65536)
    # one unit apart: M = 32768 -> LUT[32] = 5399
    np.testing.assert_array_equal(O.q16_pair(x, x - 65536), x + 32768 + 5399)
    # beyond 16 units the smaller operand vanishes exactly
    for d in (17 * 65536, 100 * 65536, 2 ** 30):
        np.testing.assert_array_equal(O.q16_pair(x, x - d), x)
    # symmetric
    rng = np.random.default_rng(0)
    a = rng.integers(-2 ** 31, 2 ** 31, 10000, dtype=np.int64).astype(np.int32)
    b = rng.integers(-2 ** 31, 2 ** 31, 10000, dtype=np.int64).astype(np.int32)
    np.testing.assert_array_equal(O.q16_pair(a, b), O.q16_pair(b, a))
    # the identity of the GPU kernels vanishes against ordinary values
    v = (rng.standard_normal(1000) * 2 ** 22).astype(np.int32)
    np.testing.assert_array_equal(O.q16_pair(v, np.full_like(v, NEG)), v)
    assert O.q16_pair(np.array([NEG], np.int32), np.array([NEG], np.int32))[0] == NEG + 65536


def test_q16_pair_error_bound_exhaustive():
    """Every gap d in [0, 17*65536]: |pair(0, -d) - 65536*log2(1 + 2^(-d/65536))|
    stays within the Mitchell+LUT bound, and without the LUT the error is the
    plain Mitchell error (up to 0.086 log2 units)."""
    d = np.arange(0, 17 * 65536 + 1, dtype=np.int64)
    zero = np.zeros(d.size, np.int32)
    exact = 65536.0 * np.log2(1.0 + np.exp2(-d / 65536.0))
    err = O.q16_pair(zero, (-d).astype(np.int32)) - exact
    assert np.max(np.abs(err)) < 0.011 * 65536, np.max(np.abs(err)) / 65536
    err_nolut = O.q16_pair(zero, (-d).astype(np.int32), mode="nolut") - exact
    assert 0.08 * 65536 < np.max(np.abs(err_nolut)) < 0.09 * 65536
    # the x86 scalar helper equals the GPU form wherever the difference does not wrap
    np.testing.assert_array_equal(O.q16_pair(zero, (-d).astype(np.int32), mode="x86"),
                                  O.q16_pair(zero, (-d).astype(np.int32)))


def test_q16_pair_wrapped_difference():
    """Operands more than 2^31 apart make the difference wrap to a positive
    value.  For a wrapped difference of 2^20 + 1 the count -(sub >> 16) is -16:
    the GPU/SIMD form reads it unsigned (>= 32 -> M = 0, the max survives), the
    x86 scalar helper shifts by -16 mod 32 = 16 (M = 1).  For a wrapped
    difference below 2^16 the count is 0 and both add 65536 + sub."""
    a = np.array([2 ** 31 - 1], np.int32)
    b = np.array([-2 ** 31 + 2 ** 20], np.int32)
    assert O.q16_pair(a, b)[0] == 2 ** 31 - 1
    assert O.q16_pair(a, b, mode="x86")[0] == -2 ** 31  # (2^31 - 1) + 1 wraps
    b2 = np.array([-2 ** 31 + 5], np.int32)  # wrapped difference 6
    want = np.int64(2 ** 31 - 1) + 65536 + 6 - 2 ** 32
    assert O.q16_pair(a, b2)[0] == want
    assert O.q16_pair(a, b2, mode="x86")[0] == want


def test_q16_luts():
    """The Q10.6 table is the Q16.16 table rounded to 6 fractional bits
    (lse_kernel_q10_6.cu:23-26)."""
    q16 = O.lut_q16()
    q10 = O.lut_q10_6()
    assert q16[0] == 0 and q16[32] == 5399 and q16[63] == 2
    np.testing.assert_array_equal(q10, np.floor(q16 / 1024.0 + 0.5).astype(np.int64))


# ---------------------------------------------------------------------------
# Q10.6 pair op
# ---------------------------------------------------------------------------
def test_q10_6_pair_closed_forms_and_bound():
    x = np.array([0, 100, -5000, 30000], np.int32)
    np.testing.assert_array_equal(O.q10_6_pair(x, x), x + 64)
    # d = 32 (half a unit): M = 48 -> LUT[48] = 1
    np.testing.assert_array_equal(O.q10_6_pair(x, x - 32), x + 49)
    for d in (17 * 64, 400, 10 ** 6):
        np.testing.assert_array_equal(O.q10_6_pair(x, x - d), x)
    d = np.arange(0, 2000, dtype=np.int64)
    zero = np.zeros(d.size, np.int32)
    exact = 64.0 * np.log2(1.0 + np.exp2(-d / 64.0))
    err = O.q10_6_pair(zero, (-d).astype(np.int32)) - exact
    assert np.max(np.abs(err)) <= 1.6, np.max(np.abs(err))  # Mitchell alone: ~5.5
    # the whole pair op depends only on the gap and is the identity past 384
    assert np.all(O.q10_6_pair(zero, (-d).astype(np.int32))[385:] == 0)
    rng = np.random.default_rng(1)
    a = rng.integers(-30000, 30000, 5000).astype(np.int32)
    b = rng.integers(-30000, 30000, 5000).astype(np.int32)
    np.testing.assert_array_equal(O.q10_6_pair(a, b), O.q10_6_pair(b, a))
    np.testing.assert_array_equal(O.q10_6_pair(a, b) - np.maximum(a, b),
                                  O.q10_6_pair(np.zeros_like(a), -np.abs(a - b)))


# ---------------------------------------------------------------------------
# quantisers
# ---------------------------------------------------------------------------
def test_q16_quantisers():
    assert float(O.Q16_CONV) == 94548.4609375
    specials = np.array([np.nan, np.inf, -np.inf, 3e5, -3e5, 0.0, -0.0], np.float32)
    np.testing.assert_array_equal(O.q16_quant(specials, "gpu"),
                                  [0, 2 ** 31 - 1, -2 ** 31, 2 ** 31 - 1, -2 ** 31, 0, 0])
    np.testing.assert_array_equal(O.q16_quant(specials, "cpu_simd")[1:],
                                  [2147483520, -2147483520, 2147483520, -2147483520, 0, 0])
    # sparse quantiser clamps logits at -20000 first; NaN -> -20000
    np.testing.assert_array_equal(O.q16_quant(np.array([np.nan, -1e9], np.float32), "sparse"),
                                  [int(np.float32(-20000.0) * O.Q16_CONV)] * 2)  # fp32 product: -1890969216
    # ties: round half to even on the GPU and in SIMD, half away from zero in the scalar CPU path
    v = np.array([2.5, 3.5, -2.5], np.float32) / O.Q16_CONV
    prod = v * O.Q16_CONV
    exact_ties = prod == np.array([2.5, 3.5, -2.5], np.float32)
    if exact_ties.all():
        np.testing.assert_array_equal(O.q16_quant(v, "gpu"), [2, 4, -2])
        np.testing.assert_array_equal(O.q16_quant(v, "cpu_scalar"), [3, 4, -3])
    # in range, GPU and CPU SIMD quantisers agree (SIMD one pinned by the reference build)
    x = (np.random.default_rng(2).standard_normal(100000) * 1000).astype(np.float32)
    np.testing.assert_array_equal(O.q16_quant(x, "gpu"), O.q16_quant(x, "cpu_simd"))


def test_to_q10_6():
    x = np.array([0.0, 1.0, -1.0, 1000.0, -1000.0, 0.5 / 92.33248], np.float32)
    q = O.to_q10_6(x)
    conv = np.float32(math.log2(math.e) * 64.0)
    assert q[1] == int(np.rint(np.float32(1.0) * conv)) == 92
    assert q[3] == 32767 and q[4] == -32768
    assert q.dtype == np.int16


# ---------------------------------------------------------------------------
# GPU reduction trees
# ---------------------------------------------------------------------------
def _chain(vals, pair):
    acc = np.array([vals[0]], np.int32)
    for v in vals[1:]:
        acc = pair(acc, np.array([v], np.int32))
    return int(acc[0])


def test_gpu_tree_single_chain_row():
    """N=4, aligned: only virtual thread 0 has elements; every other lane holds
    the identity, which vanishes, so the row equals the sequential chain."""
    q = np.array([[1000000, -300000, 2500000, 2400000]], np.int32)
    out, raw = O.q16_gpu_rows(q, raw=True)
    assert raw[0] == _chain(list(q[0]), O.q16_pair)
    assert out[0] == np.float32(np.float32(raw[0]) * O.Q16_OUT)


def test_gpu_tree_equal_rows_closed_form():
    """N = 256*4*k equal values v: each of the 256 chains folds 4k copies
    (chain value c), then 8 doubling levels (5 in the warp, 3 in the final
    stage where the identity padding drops out): result c + 8*65536."""
    for k in (1, 2, 3):
        v = 123456
        q = np.full((1, 1024 * k), v, np.int32)
        raw = O.q16_gpu_rows(q, raw=True)[1][0]
        c = _chain([v] * (4 * k), O.q16_pair)
        assert raw == c + 8 * 65536
    # the same for Q10.6 with +64 per level
    q = np.full((1, 2048), 300, np.int16)
    raw = O.q10_6_rows(q, raw=True)[1][0]
    assert raw == _chain([300] * 8, O.q10_6_pair) + 8 * 64


def test_gpu_tree_prefix_and_suffix():
    """A misaligned row start gives threads 0..p-1 one prefix element; the
    remaining elements form vector chunks and a suffix.  With N = 7 and a row
    starting 4 bytes past a 16-byte boundary: prefix 3 (threads 0,1,2), one
    chunk (thread 0) and no suffix: thread 0 = chain(e0, e3..e6), threads 1, 2
    hold e1, e2; the warp butterfly then pairs lanes (0,2) at distance 2 and
    (0,1) at distance 1."""
    q = np.array([[40000, -70000, 90000, 10000, 20000, 30000, 40000]], np.int32)
    raw = O.q16_gpu_rows(q, base_mod=4, raw=True)[1][0]
    p = O.q16_pair
    t0 = _chain([q[0, 0], q[0, 3], q[0, 4], q[0, 5], q[0, 6]], p)
    one = lambda a, b: int(p(np.array([a], np.int32), np.array([b], np.int32))[0])  # noqa: E731
    # off=16,8,4: lanes 0..2 pair with identity lanes (exact); lane 0 then
    # pairs with lane 2 (off=2) and the result with lane 1's (lane1 paired with lane3 = identity)
    want = one(one(t0, int(q[0, 2])), int(q[0, 1]))
    assert raw == want
    # aligned start: the same 7 values take one chunk (thread 0: e0..e3) and a suffix (threads 0..2)
    raw_al = O.q16_gpu_rows(q, base_mod=0, raw=True)[1][0]
    t0 = _chain([q[0, 0], q[0, 1], q[0, 2], q[0, 3], q[0, 4]], p)
    want_al = one(one(t0, int(q[0, 6])), int(q[0, 5]))
    assert raw_al == want_al


def _one(pair, a, b):
    return int(pair(np.array([a], np.int32), np.array([b], np.int32))[0])


@pytest.mark.parametrize("kind", ["q16", "q10_6"])
def test_gpu_tree_chunk_striding(kind):
    """Chunk-to-thread striding of the GPU trees (lse_kernel.cu:110,
    lse_kernel_q10_6.cu:96): virtual thread t folds chunks t, t+256, t+512, ...
    in ascending order, each chunk's elements in x, y, z, w order.

    An aligned row of N = 3072 has 768 four-element chunks.  Every element is a
    filler far below the rest (more than 16 units of the format, also after the
    fillers' own chains and butterflies), so each pair with a filler is exact,
    except for five values: A at chunk 0, B at chunk 256, D and D2 at elements
    0 and 3 of chunk 512 (all thread 0) and C at chunk 1 (thread 1).  Thread 0
    is then chain(A, B, D, D2); threads 0 and 1 meet at the butterfly's last
    warp level and the other lanes carry fillers or the identity, so the row is
    pair(chain(A, B, D, D2), C).  The expected value is computed by hand from
    the pair op; the alternatives a plausible slip would give (descending chunk
    order, chunk elements in w..x order, contiguous thread ranges: thread 0 =
    {A, C}, thread 85 = {B}, thread 170 = {D, D2}) are checked to differ."""
    if kind == "q16":
        pair, dt, filler = O.q16_pair, np.int32, -50 * 65536
        A, B, D, D2, C = 124043, 134170, 197962, 249158, 9136
    else:
        pair, dt, filler = O.q10_6_pair, np.int16, -20000
        A, B, D, D2, C = 202, 137, 89, 137, 114
    row = np.full(3072, filler, dt)
    row[4 * 0] = A
    row[4 * 256] = B
    row[4 * 512] = D
    row[4 * 512 + 3] = D2
    row[4 * 1] = C
    raw = (O.q16_gpu_rows if kind == "q16" else O.q10_6_rows)(row[None, :], raw=True)[1][0]

    def chain(vals):
        acc = vals[0]
        for v in vals[1:]:
            acc = _one(pair, acc, v)
        return acc

    want = _one(pair, chain([A, B, D, D2]), C)
    wrong = {
        "descending chunks": _one(pair, chain([D2, D, B, A]), C),
        "chunk elements w..x": _one(pair, chain([A, B, D2, D]), C),
        "contiguous threads": _one(pair, _one(pair, _one(pair, A, C), B), chain([D, D2])),
    }
    assert all(v != want for v in wrong.values()), wrong
    assert raw == want, (raw, want, wrong)


# Published envelopes: intlse_gpu / intlse_nolut / intlse_cpu mean |err| vs fp64
# at B=512, 20 seeds, inputs U(lo, 0) (experiment_microbenchmark/microbench/
# outputs/benchmark_results.json, ranges U(-1,0), U(-100,0), U(-500,0)).
ENVELOPE = {
    # (lo, N): (intlse_gpu, intlse_nolut, intlse_cpu)
    (-1, 1024): (8.86e-05, 0.0905, 0.00015),
    (-1, 8192): (0.00196, 0.262, 5.57e-05),
    (-1, 32000): (0.114, 0.305, 5.2e-05),
    (-1, 128256): (0.269, 0.321, 6.4e-05),
    (-100, 4096): (0.0012, 0.168, 0.00118),
    (-100, 128256): (0.0109, 0.234, 0.00111),
    (-500, 16384): (0.00123, 0.167, 0.0012),
    (-500, 128256): (0.00232, 0.178, 0.00114),
}


@pytest.mark.parametrize("lo,N", sorted(ENVELOPE))
def test_gpu_tree_matches_published_envelope(lo, N):
    rng = np.random.default_rng(N + int(-lo))
    B = 256 if N > 20000 else 512
    x = (rng.random((B, N), dtype=np.float32) * np.float32(-lo) + np.float32(lo)).astype(np.float32)
    ref = O.fp64_lse_ref(x)
    gpu, nolut, cpu = ENVELOPE[(lo, N)]
    e_gpu = np.abs(O.q16_gpu_rows(x) - ref).mean()
    e_nolut = np.abs(O.q16_gpu_rows(x, use_lut=False) - ref).mean()
    assert abs(e_gpu / gpu - 1) < 0.2, (e_gpu, gpu)
    assert abs(e_nolut / nolut - 1) < 0.2, (e_nolut, nolut)
    if N <= 8192:
        e_cpu = np.abs(O.intlse_cpu_rows(x, True) - ref).mean()
        assert abs(e_cpu / cpu - 1) < 0.25, (e_cpu, cpu)


# Reduced-bit envelope: Q10.6 mean |err| vs fp64 at B=512, U(-100, 0)
# (experiment_microbenchmark/reduced_bit/outputs/bench_results.json).
Q106_ENVELOPE = {64: 0.01135, 1024: 0.02728, 16384: 0.04471, 128256: 0.09466}


@pytest.mark.parametrize("N", sorted(Q106_ENVELOPE))
def test_q10_6_tree_matches_published_envelope(N):
    rng = np.random.default_rng(N)
    B = 128 if N > 20000 else 512
    x = (rng.random((B, N), dtype=np.float32) * np.float32(100.0) - np.float32(100.0)).astype(np.float32)
    out = O.q10_6_rows(O.to_q10_6(x))
    e = np.abs(out - O.fp64_lse_ref(x)).mean()
    assert abs(e / Q106_ENVELOPE[N] - 1) < 0.2, (e, Q106_ENVELOPE[N])


# ---------------------------------------------------------------------------
# sparse Q16 tree
# ---------------------------------------------------------------------------
def test_edge_thread_rule():
    assert [O.edge_threads(k) for k in (1, 8, 9, 16, 17, 32, 33, 256)] == [1, 1, 2, 2, 4, 4, 8, 8]


def test_sparse_q16_closed_forms():
    """One edge: the identity seed vanishes -> q itself.  Two equal edges
    (ET=1): pair(q, q) = q + 65536.  Nine equal edges (ET=2): chains of 5 and 4
    then one butterfly level."""
    child = np.array([[1.25, -3.0], [0.5, 0.75]], np.float32)  # 2 children x batch 2
    for k in (1, 2, 9):
        off = np.array([0, k], np.int64)
        cids = np.zeros(k, np.int32)
        lp = np.full(k, -0.5, np.float32)
        out = O.sparse_q16_csr(child, off, cids, lp)
        for b in range(2):
            q = int(O.q16_quant(np.array([np.float32(-0.5) + child[0, b]], np.float32), "sparse")[0])
            if k == 1:
                r = q
            elif k == 2:
                r = q + 65536
            else:
                c5 = _chain([q] * 5, O.q16_pair)
                c4 = _chain([q] * 4, O.q16_pair)
                r = int(O.q16_pair(np.array([c5], np.int32), np.array([c4], np.int32))[0])
            assert out[0, b] == np.float32(np.float32(r) * O.Q16_OUT)
    # an empty node gives -inf
    out = O.sparse_q16_csr(child, np.array([0, 0], np.int64), np.zeros(0, np.int32), np.zeros(0, np.float32))
    assert np.all(np.isneginf(out))


def test_sparse_q16_edge_striding():
    """Edge-to-chain striding of the sparse Q16 tree (sparse_q16_kernel.cu:110):
    with fan-in 9 there are ET = 2 chains, chain c folding edges c, c+2, c+4, ...
    in ascending order from the identity seed.  Edges 0, 1, 2 and 4 carry
    values; the other edges are fillers 100 nats lower, whose pairs are exact.
    So chain 0 = chain(a0, a2, a4), chain 1 = a1, and the node is
    pair(chain 0, chain 1).  A contiguous split (chain 0 = edges 0..4) would give
    chain(a0, a1, a2, a4), and a descending walk chain(a4, a2, a0) paired with
    a1; both are checked to differ."""
    vals = np.full(9, -100.0, np.float32)
    vals[[0, 1, 2, 4]] = np.array([-1.25, -0.5, -0.25, 0.375], np.float32)
    child = vals[:, None].copy()  # 9 children x batch 1, one child per edge
    lp = np.full(9, -0.5, np.float32)
    out = O.sparse_q16_csr(child, np.array([0, 9], np.int64), np.arange(9, dtype=np.int32), lp)
    q = [int(O.q16_quant(np.array([vals[e] + lp[e]], np.float32), "sparse")[0]) for e in range(9)]
    p = O.q16_pair

    def chain(vs):
        acc = vs[0]
        for v in vs[1:]:
            acc = _one(p, acc, v)
        return acc

    want = _one(p, chain([q[0], q[2], q[4]]), q[1])
    wrong = {"contiguous": chain([q[0], q[1], q[2], q[4]]),
             "descending": _one(p, chain([q[4], q[2], q[0]]), q[1])}
    assert all(v != want for v in wrong.values()), wrong
    assert out[0, 0] == np.float32(np.float32(want) * O.Q16_OUT), (out[0, 0], want, wrong)
    # the block layout walks the same chains
    nm = O.sparse_q16_blocked(np.zeros((1, 1), np.float32), child, lp.reshape(1, 1, 9),
                              np.array([0], np.int64), np.arange(9, dtype=np.int64).reshape(1, 9), 1)
    assert nm[0, 0] == out[0, 0]


def test_sparse_q16_tracks_float_oracle():
    rng = np.random.default_rng(5)
    nodes, nch, batch = 300, 200, 16
    k = O.powerlaw_fanin(nodes, seed=1)
    off = np.concatenate([[0], np.cumsum(k)]).astype(np.int64)
    cids = rng.integers(0, nch, off[-1]).astype(np.int32)
    lp = np.log(rng.random(off[-1])).astype(np.float32)
    child = np.log(rng.random((nch, batch))).astype(np.float32)
    want = O.sparse_csr_fp64(child, off, cids, lp)
    got = O.sparse_q16_csr(child, off, cids, lp)
    err = np.abs(got - want)
    assert err.mean() < 5e-3 and err.max() < 0.05, (err.mean(), err.max())


def test_sparse_blocked_q16_equals_csr_on_expanded_layout():
    """The pyjuice block layout is the CSR layout after block expansion
    (run_pyjuice.py:103-113): node nids[j]+p owns edges cids[j, :] with
    weights params[pids[j, e] + p]."""
    rng = np.random.default_rng(6)
    nb, ne, bs, batch, nelem = 3, 5, 4, 8, 20
    nids = np.array([0, 4, 8], np.int64)
    cids = rng.integers(0, nelem, (nb, ne)).astype(np.int64)
    pids = rng.integers(0, 40, (nb, ne)).astype(np.int64)
    params = rng.random(64).astype(np.float32)
    em = np.log(rng.random((nelem, batch))).astype(np.float32)
    logw = np.empty((nb, bs, ne), np.float32)
    for j in range(nb):
        for p in range(bs):
            logw[j, p] = np.log(np.maximum(params[pids[j] + p], np.float32(1e-45)))
    nm = O.sparse_q16_blocked(np.zeros((12, batch), np.float32), em, logw, nids, cids, bs)
    off = np.arange(0, nb * bs * ne + 1, ne, dtype=np.int64)
    ccs = np.repeat(cids, bs, axis=0).reshape(-1).astype(np.int32)
    out = O.sparse_q16_csr(em, off, ccs, logw.reshape(-1))
    np.testing.assert_array_equal(nm, out)


# ---------------------------------------------------------------------------
# float oracles
# ---------------------------------------------------------------------------
def test_lse_fp64_against_scipy_and_invariants():
    from scipy.special import logsumexp

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((50, 333)) * 5).astype(np.float32)
    np.testing.assert_allclose(O.lse_fp64(x), logsumexp(x.astype(np.float64), axis=-1), rtol=1e-13)
    np.testing.assert_allclose(O.lse_fp64(x.astype(np.float64) + 7.0), O.lse_fp64(x) + 7.0, rtol=1e-12)
    np.testing.assert_allclose(O.lse_fp64(np.full((2, 1000), 2.0)), 2.0 + np.log(1000.0), rtol=1e-14)
    np.testing.assert_allclose(O.lse_fp64(x[:, rng.permutation(333)]), O.lse_fp64(x), rtol=1e-13)
    # N = 2: textbook max + log1p(exp(-|a - b|))
    a, b = 3.0, -1.5
    assert math.isclose(O.lse_fp64(np.array([[a, b]]))[0], a + math.log1p(math.exp(-(a - b))), rel_tol=1e-15)


def test_lse_fp64_special_values_follow_torch():
    import torch

    x = O.make_robust_rows(O.make_c2_input(12, 50, seed=2), seed=3)
    want = torch.logsumexp(torch.from_numpy(x).double(), -1).numpy()
    np.testing.assert_allclose(O.lse_fp64(x), want, rtol=1e-12, equal_nan=True)


def test_lse_bwd_fp64_is_scaled_softmax():
    from scipy.special import softmax

    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 40))
    g = rng.standard_normal(7)
    np.testing.assert_allclose(O.lse_bwd_fp64(g, x, O.lse_fp64(x)), g[:, None] * softmax(x, axis=-1), rtol=1e-12)


def test_fuselse_cpu_port_envelope_and_pair():
    """Sequential float pair chain (fused_fp32_cpu.cpp): N=2 is the textbook
    pair in fp32, and at N=128256 on U(-100,0) the chain's mean |err| lands on
    the published 1.06e-4 (benchmark_results.json fuselse_cpu)."""
    x = np.array([[3.0, -1.5]], np.float32)
    want = np.float32(3.0) + np.log1p(np.exp(np.float32(-4.5)))
    assert abs(O.fuselse_cpu_rows(x)[0] - want) <= 2e-7
    rng = np.random.default_rng(8)
    x = (rng.random((64, 128256), dtype=np.float32) * np.float32(100.0) - np.float32(100.0))
    e = np.abs(O.fuselse_cpu_rows(x) - O.fp64_lse_ref(x)).mean()
    assert abs(e / 1.06e-4 - 1) < 0.25, e


def _same_bits(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.int32), want[ok].view(np.int32))


def test_fuselse_cpu_port_matches_reference_fixture():
    """The C port equals the reference's own cpu_lse_float bit for bit on the
    fixture tests/golden/make_golden.py wrote from the compiled reference
    (fuselse/cpu/fused_fp32_cpu.cpp built by oracle/Makefile): the C1 shapes,
    a C2-style sample, N = 1..3 and special-value rows."""
    d = np.load(os.path.join(GOLD, "fuselse_cpu_ref.npz"))
    xo = oo = 0
    for B, N in d["shapes"]:
        x = d["x"][xo:xo + int(B * N)].reshape(int(B), int(N))
        want = d["out"][oo:oo + int(B)]
        xo += int(B * N)
        oo += int(B)
        _same_bits(O.fuselse_cpu_rows(x), want)
    assert xo == d["x"].size and oo == d["out"].size


@pytest.mark.skipif(not O.ref_fuselse_available(), reason="reference FuseLSE-CPU build (oracle/_ref) absent")
@pytest.mark.parametrize("B,N,scale", [(3, 2, 1.0), (16, 4097, 3.0), (8, 128256, 3.0), (5, 1000, 80.0)])
def test_fuselse_cpu_port_matches_compiled_reference(B, N, scale):
    x = (np.random.default_rng(B * N).standard_normal((B, N), dtype=np.float32) * np.float32(scale))
    _same_bits(O.fuselse_cpu_rows(x), O.ref_fuselse_cpu(x))


# ---------------------------------------------------------------------------
# selective log-softmax (trl.trainer.utils.selective_log_softmax, fp32 branch)
# ---------------------------------------------------------------------------
def test_selective_logsoftmax_fp64_against_scipy_and_closed_forms():
    from scipy.special import log_softmax

    rng = np.random.default_rng(12)
    x = (rng.standard_normal((40, 257)) * 4).astype(np.float32)
    idx = rng.integers(0, 257, 40)
    logp, lse = O.selective_logsoftmax_fp64(x, idx)
    want = np.take_along_axis(log_softmax(x.astype(np.float64), axis=-1), idx[:, None], axis=-1)[:, 0]
    np.testing.assert_allclose(logp, want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, O.lse_fp64(x), rtol=0)
    # the probabilities of all targets of a row sum to one
    allp = np.stack([O.selective_logsoftmax_fp64(x[:3], np.full(3, t))[0] for t in range(257)], axis=1)
    np.testing.assert_allclose(np.exp(allp).sum(axis=1), 1.0, rtol=1e-12)
    # N = 2: logp of the first of (a, b) is -log1p(exp(b - a))
    a, b = 1.25, -2.0
    lp, _ = O.selective_logsoftmax_fp64(np.array([[a, b]]), np.array([0]))
    assert math.isclose(lp[0], -math.log1p(math.exp(b - a)), rel_tol=1e-13)
    # an index outside [0, N) gives NaN
    lp, _ = O.selective_logsoftmax_fp64(x[:4], np.array([-1, 257, 3, 10 ** 9]))
    assert np.isnan(lp[0]) and np.isnan(lp[1]) and not np.isnan(lp[2]) and np.isnan(lp[3])


def test_selective_logsoftmax_bwd_fp64_against_finite_differences_and_torch():
    import torch

    rng = np.random.default_rng(13)
    x = rng.standard_normal((3, 9)) * 2
    idx = np.array([0, 4, 8])
    g = rng.standard_normal(3)
    _, lse = O.selective_logsoftmax_fp64(x, idx)
    got = O.selective_logsoftmax_bwd_fp64(g, x, idx, lse)
    # central differences of sum_r g[r] * logp[r]
    h = 1e-6
    fd = np.zeros_like(x)
    for r in range(3):
        for i in range(9):
            xp, xm = x.copy(), x.copy()
            xp[r, i] += h
            xm[r, i] -= h
            fp = (g * O.selective_logsoftmax_fp64(xp, idx)[0]).sum()
            fm = (g * O.selective_logsoftmax_fp64(xm, idx)[0]).sum()
            fd[r, i] = (fp - fm) / (2 * h)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(got.sum(axis=1), 0.0, atol=1e-12)
    xt = torch.from_numpy(x).requires_grad_(True)
    lp = torch.log_softmax(xt, -1).gather(-1, torch.from_numpy(idx)[:, None])[:, 0]
    (lp * torch.from_numpy(g)).sum().backward()
    np.testing.assert_allclose(got, xt.grad.numpy(), rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("dtype", ["float32", "float64", "bfloat16"])
def test_trl_algorithm_fallback_matches_oracle(dtype):
    """The package's restatement of trl's algorithm, used for inputs the kernels
    do not take, against the fp64 oracle on the CPU."""
    import torch

    from fuselse_amd.selective import _trl_algorithm

    rng = np.random.default_rng(14)
    x = (rng.standard_normal((2, 5, 300)) * 3).astype(np.float32)
    idx = rng.integers(0, 300, (2, 5))
    xt = torch.from_numpy(x).to(getattr(torch, dtype))
    got = _trl_algorithm(xt, torch.from_numpy(idx)).double().numpy()
    want, _ = O.selective_logsoftmax_fp64(xt.double().numpy().reshape(10, 300), idx.reshape(10))
    tol = 2e-2 if dtype == "bfloat16" else 1e-5
    np.testing.assert_allclose(got.reshape(10), want, rtol=tol, atol=tol)


# ---------------------------------------------------------------------------
# sparse CSR backward (flows)
# ---------------------------------------------------------------------------
def _tiny_csr(rng, nodes, children, batch, max_fan=6, empty_node=True):
    fan = rng.integers(1, max_fan + 1, nodes)
    if empty_node:
        fan[1] = 0
    off = np.concatenate([[0], np.cumsum(fan)]).astype(np.int64)
    cid = rng.integers(0, children, int(off[-1]))
    lw = rng.standard_normal(int(off[-1]))
    child = rng.standard_normal((children, batch)) * 2
    return off, cid, lw, child


def test_sparse_csr_bwd_fp64_against_torch_autograd_and_closed_forms():
    import torch

    rng = np.random.default_rng(31)
    off, cid, lw, child = _tiny_csr(rng, 9, 7, 5)
    child[3, 2] = -np.inf                      # a -inf child value contributes 0
    out = O.sparse_csr_fp64(child, off, cid, lw)
    gout = rng.standard_normal(out.shape)
    gc, gl = O.sparse_csr_bwd_fp64(child, out, gout, off, cid, lw)
    # torch fp64 autograd of the same layer written with gather + logsumexp
    ct = torch.from_numpy(np.where(np.isneginf(child), -1e300, child)).requires_grad_(True)
    lt = torch.from_numpy(lw).requires_grad_(True)
    rows = []
    for n in range(9):
        a, b = off[n], off[n + 1]
        if a == b:
            rows.append(torch.full((5,), -1e300, dtype=torch.float64))
            continue
        rows.append(torch.logsumexp(lt[a:b, None] + ct[torch.from_numpy(cid[a:b])], dim=0))
    yt = torch.stack(rows)
    (yt * torch.from_numpy(np.where(np.isneginf(out), 0.0, gout))).sum().backward()
    np.testing.assert_allclose(gc, ct.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(gl, lt.grad.numpy(), rtol=1e-12, atol=1e-14)
    # the softmax weights of a node's edges sum to one per column, so the
    # log-weight gradients of a node sum to the node's gradient over the batch
    for n in range(9):
        a, b = off[n], off[n + 1]
        if a < b:
            assert math.isclose(gl[a:b].sum(), gout[n].sum(), rel_tol=1e-12, abs_tol=1e-12)


def test_sparse_csr_bwd_fp64_finite_differences():
    rng = np.random.default_rng(32)
    off, cid, lw, child = _tiny_csr(rng, 4, 5, 3, empty_node=False)
    gout = rng.standard_normal((4, 3))

    def f(ch, l):
        return (gout * O.sparse_csr_fp64(ch, off, cid, l)).sum()

    out = O.sparse_csr_fp64(child, off, cid, lw)
    gc, gl = O.sparse_csr_bwd_fp64(child, out, gout, off, cid, lw)
    h = 1e-6
    for c in range(5):
        for b in range(3):
            p, m = child.copy(), child.copy()
            p[c, b] += h
            m[c, b] -= h
            assert math.isclose(gc[c, b], (f(p, lw) - f(m, lw)) / (2 * h), rel_tol=1e-6, abs_tol=1e-8)
    for e in range(len(lw)):
        p, m = lw.copy(), lw.copy()
        p[e] += h
        m[e] -= h
        assert math.isclose(gl[e], (f(child, p) - f(child, m)) / (2 * h), rel_tol=1e-6, abs_tol=1e-8)


# ---------------------------------------------------------------------------
# the reference's CPU wrappers (lse_ctypes_wrapper.py:99-125, torch_wrapper.py:9-29)
# ---------------------------------------------------------------------------
@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("shape,axis,keepdims", [((300,), None, False), ((300,), -1, True), ((4, 130), -1, False),
                                                  ((4, 130), 1, True), ((2, 3, 70), -1, False), ((2, 3, 70), None, True)])
def test_cpu_wrapper_port_equals_compiled_reference(shape, axis, keepdims):
    """The wrapper restated over the C port gives the same bits as over the
    compiled reference kernel, for every dispatch branch."""
    rng = np.random.default_rng(sum(shape))
    a = (rng.standard_normal(shape) * 4).astype(np.float32)
    a.flat[3] = -np.inf                       # the -inf-identity variant
    got = O.logsumexp_intlse(a, axis=axis, keepdims=keepdims, backend="port")
    want = O.logsumexp_intlse(a, axis=axis, keepdims=keepdims, backend="ref")
    assert type(got) is type(want)
    np.testing.assert_array_equal(np.asarray(got), np.asarray(want))
    if keepdims and axis is not None:
        assert np.asarray(got).ndim == len(shape)
    if axis is None:
        # the reference's finite full reduction returns a float whatever keepdims says
        assert isinstance(got, float)


# NaN and +inf inputs take np.logaddexp.reduce, as the reference's wrapper does;
# numpy warns on the NaN it produces from inf - inf
@pytest.mark.filterwarnings("ignore:invalid value encountered in reduce:RuntimeWarning")
def test_cpu_wrapper_special_values_and_axes():
    from scipy.special import logsumexp

    rng = np.random.default_rng(3)
    a = rng.standard_normal((3, 50)).astype(np.float32)
    # NaN / +inf anywhere: the whole call goes to np.logaddexp.reduce
    b = a.copy()
    b[1, 7] = np.inf
    r = O.logsumexp_intlse(b, axis=-1)
    np.testing.assert_array_equal(r, np.logaddexp.reduce(b, axis=-1))
    assert r[1] == np.inf
    b[2, 3] = np.nan
    assert np.isnan(O.logsumexp_intlse(b))
    assert O.logsumexp_intlse(b, axis=None, keepdims=True).shape == (1, 1)
    # finite rows go through the fixed-point kernel (its ~0.03 nat error at
    # N = 50 is pinned by the envelope tests above)
    np.testing.assert_allclose(O.logsumexp_intlse(a, axis=-1), logsumexp(a.astype(np.float64), axis=-1), atol=0.05)
    np.testing.assert_array_equal(O.logsumexp_intlse(a, axis=-1), O.intlse_cpu_rows(a, True))
    assert isinstance(O.logsumexp_intlse(a[0]), float)
    with pytest.raises(NotImplementedError):
        O.logsumexp_intlse(a, axis=0)


def test_cpu_torch_wrapper_dispatch():
    import torch

    x = torch.randn(4, 40)
    got = O.logsumexp_intlse_torch(x, dim=-1)
    assert got.dtype == torch.float32 and got.shape == (4,)
    np.testing.assert_array_equal(got.numpy(), O.intlse_cpu_rows(x.numpy(), True))
    assert O.logsumexp_intlse_torch(x, dim=1, keepdim=True).shape == (4, 1)
    # fallbacks to torch.logsumexp: grad, dtype, dim, N < 2
    xg = x.clone().requires_grad_(True)
    torch.testing.assert_close(O.logsumexp_intlse_torch(xg, -1), torch.logsumexp(xg, -1))
    torch.testing.assert_close(O.logsumexp_intlse_torch(x.double(), -1), torch.logsumexp(x.double(), -1))
    torch.testing.assert_close(O.logsumexp_intlse_torch(x, 0), torch.logsumexp(x, 0))
    torch.testing.assert_close(O.logsumexp_intlse_torch(x[:, :1], -1), torch.logsumexp(x[:, :1], -1))
    assert isinstance(O.logsumexp_intlse_torch(torch.randn(30), -1), torch.Tensor)


def test_sparse_blocked_bwd_fp64_against_csr_expansion_and_autograd():
    """The block-layout flows equal the CSR flows of the layer expanded to one
    node per (block, position), and torch fp64 autograd of the block-layout
    forward written with gather + logsumexp."""
    import torch

    rng = np.random.default_rng(41)
    nb, ne, bs, batch, nel, npar = 3, 4, 2, 5, 6, 20
    nids = np.array([0, 2, 4], np.int64)
    cids = rng.integers(0, nel, (nb, ne)).astype(np.int64)
    cids[0, :2] = 1                                  # repeated child in one block
    pids = rng.integers(0, npar - bs, (nb, ne)).astype(np.int64)
    params = rng.random(npar) + 1e-3
    em = np.log(rng.random((nel, batch)))
    em[2, 1] = -np.inf
    rows, vals = O.sparse_blocked_fp64(em, params, nids, cids, pids, bs)
    nm = np.zeros((nb * bs, batch))
    nm[rows] = vals
    nf = rng.standard_normal(nm.shape)
    de, dp = O.sparse_blocked_bwd_fp64(nf, nm, em, params, nids, cids, pids, bs)
    # CSR expansion: node (j, p) -> row nids[j] + p, edges e in order
    off = np.arange(nb * bs + 1, dtype=np.int64) * ne
    cid = np.repeat(cids[:, None, :], bs, axis=1).reshape(-1)
    q = (pids[:, None, :] + np.arange(bs)[None, :, None]).reshape(-1)
    lw = np.log(np.maximum(params[q], 1e-45))
    order_rows = (nids[:, None] + np.arange(bs)[None, :]).reshape(-1)
    gc, gl = O.sparse_csr_bwd_fp64(em, nm[order_rows], nf[order_rows], off, cid, lw)
    np.testing.assert_allclose(de, gc, rtol=1e-12, atol=1e-14)
    want_p = np.zeros(npar)
    np.add.at(want_p, q, gl)
    np.testing.assert_allclose(dp, want_p, rtol=1e-12, atol=1e-14)
    # torch autograd of the forward: d(sum nf * out) / d em and d / d params
    et = torch.from_numpy(np.where(np.isneginf(em), -1e300, em)).requires_grad_(True)
    pt = torch.from_numpy(params).requires_grad_(True)
    loss = 0.0
    for j in range(nb):
        for p in range(bs):
            lwt = torch.log(pt[torch.from_numpy(pids[j] + p)])
            y = torch.logsumexp(lwt[:, None] + et[torch.from_numpy(cids[j])], dim=0)
            loss = loss + (y * torch.from_numpy(nf[nids[j] + p])).sum()
    loss.backward()
    np.testing.assert_allclose(de, et.grad.numpy(), rtol=1e-12, atol=1e-14)
    # param flows are d loss / d log w = w * d loss / d w
    np.testing.assert_allclose(dp, params * pt.grad.numpy(), rtol=1e-12, atol=1e-14)
