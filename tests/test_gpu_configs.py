"""Every benchmark configuration at its full size on the GPU.

Sizes the oracle finishes in seconds are compared bit for bit.  The
60M-vector training sample and the 200M-vector encode stream are checked
through properties that hold at any size: codes equal the oracle's on a
sample, each centroid equals the serial fp32 mean of the points the previous
codebook assigned to it, WCSS does not increase, and the stream's codes
cover every vector.
"""
import time

import numpy as np
import pytest

from oracle import binding as orc
from tac_gpu import device, pq, synth

NEVER = float("-inf")
pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1).view(np.uint32)


def _log(msg):
    print(f"[configs] {msg}", flush=True)


def _serial_mean(points):
    """Centroid rule of src/tac/kmeans.zig:191-199: fp32 sums folded in
    ascending row order from 0.0, times fl(1 / fl(count)).  np.cumsum
    accumulates sequentially (np.sum would sum pairwise).  The reference
    checks the same invariant at small size (kmeans.zig:545-626)."""
    s = np.cumsum(points, axis=0, dtype=np.float32)[-1]
    return s * (np.float32(1.0) / np.float32(len(points)))


def _check_train_encode(x, w, init, ref, ref_codes):
    """tac_pq_train_encode_device on the same input: the codebooks and every
    code equal the oracle's train and encode (storage.build's chain,
    src/index/storage.zig:380-401)."""
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((w.n, w.m), pq.code_dtype(w.ksub))
    device.train_encode_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, dcodes, w.iters, NEVER)
    cb, codes = dcb.to_host(), dcodes.to_host()
    for a in (dx, dinit, dcb, dcodes):
        a.free()
    assert np.array_equal(_bits(cb), _bits(ref.codebooks))
    diff = int(np.count_nonzero(codes != ref_codes))
    _log(f"{w.name}: train+encode entry, {diff} of {codes.size} codes differ")
    assert diff == 0


@pytest.fixture(scope="module")
def corpus():
    return synth.residuals(synth.WORKLOADS["corpus-1.52m"])


def test_headline_corpus_as_benchmarked(gpu, corpus):
    """The benchmark's workload as the benchmark runs it: all 1,521,797 x 64
    residuals resident on the device, m16 k256, seeded-shuffle init, exactly
    20 Lloyd iterations (tac_pq_train_device), then encode of every vector
    (tac_pq_encode_device).  The codebooks after every iteration and all
    24.3M codes equal the oracle's bit for bit (storage.build trains, then
    encodes every token: src/index/storage.zig:380-401).  Near ties of the
    final encode (best vs second within 1e-5 relative) are counted."""
    w = synth.WORKLOADS["corpus-1.52m"]
    x = corpus
    init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((w.n, w.m), np.uint8)
    t0 = time.perf_counter()
    stats = device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER,
                                trace=True)
    device.encode_device(dx, w.n, w.dim, w.m, w.ksub, dcb, dcodes)
    device.synchronize()
    t1 = time.perf_counter()
    cb, codes = dcb.to_host(), dcodes.to_host()
    for a in (dx, dinit, dcb, dcodes):
        a.free()
    ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=w.iters, tol=NEVER,
                       n_threads=16, trace=True)
    t2 = time.perf_counter()
    assert ref.status == 0
    for t in range(w.iters):
        diff = np.count_nonzero(_bits(stats[3][t]) != _bits(ref.trace[t]))
        assert diff == 0, f"iteration {t}: {diff} codebook floats differ"
    assert np.array_equal(_bits(cb), _bits(ref.codebooks))
    assert np.all(stats[0] == w.iters)
    ref_codes = orc.pq_encode(x, w.dim, w.m, w.ksub, ref.codebooks, n_threads=16)
    t3 = time.perf_counter()
    _check_train_encode(x, w, init, ref, ref_codes)
    diff = int(np.count_nonzero(codes != ref_codes))
    ties = orc.pq_near_ties(x, w.dim, w.m, w.ksub, ref.codebooks, 1e-5, n_threads=16)
    _log(f"headline: GPU train+encode {t1 - t0:.3f} s (first call), oracle train {t2 - t1:.1f} s, "
         f"encode {t3 - t2:.1f} s; {diff} of {codes.size} codes differ; near ties {ties}")
    assert diff == 0


@pytest.mark.timeout(300)
@pytest.mark.parametrize("name", ["corpus-1.52m-m32d2", "corpus-1.52m-m8d8",
                                  "corpus-1.52m-k1024"])
def test_subspace_shape_sweep_full_corpus(gpu, corpus, name):
    """(m=32, dsub=2), (m=8, dsub=8) and (m=16, ksub=1024) on all 1,521,797
    residuals, as the benchmark runs them: resident input, 20 Lloyd
    iterations from seeded-shuffle codebooks (tac_pq_train_device), then
    encode of every vector (tac_pq_encode_device; u16 codes at ksub 1024).
    Every iteration's codebook and all codes equal the oracle's bit for bit."""
    w = synth.WORKLOADS[name]
    x = corpus
    init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
    _log(f"{name}: n={w.n} m={w.m} ksub={w.ksub} iters={w.iters}")
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((w.n, w.m), pq.code_dtype(w.ksub))
    t0 = time.perf_counter()
    stats = device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER,
                                trace=True)
    device.encode_device(dx, w.n, w.dim, w.m, w.ksub, dcb, dcodes)
    device.synchronize()
    t1 = time.perf_counter()
    cb, codes = dcb.to_host(), dcodes.to_host()
    for a in (dx, dinit, dcb, dcodes):
        a.free()
    ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=w.iters, tol=NEVER,
                       n_threads=16, trace=True)
    t2 = time.perf_counter()
    assert ref.status == 0
    for t in range(w.iters):
        diff = np.count_nonzero(_bits(stats[3][t]) != _bits(ref.trace[t]))
        assert diff == 0, f"{name} iteration {t}: {diff} codebook floats differ"
    assert np.array_equal(_bits(cb), _bits(ref.codebooks))
    assert np.all(stats[0] == w.iters)
    ref_codes = orc.pq_encode(x, w.dim, w.m, w.ksub, ref.codebooks, n_threads=16)
    assert ref_codes.dtype == codes.dtype
    _check_train_encode(x, w, init, ref, ref_codes)
    diff = int(np.count_nonzero(codes != ref_codes))
    _log(f"{name}: GPU {t1 - t0:.2f} s, oracle train {t2 - t1:.1f} s, encode "
         f"{time.perf_counter() - t2:.1f} s; {diff} of {codes.size} codes differ")
    assert diff == 0


def test_convergence_and_wcss_full_corpus(gpu, corpus):
    """The reference's defaults at full size: tol 1e-4 needs the serial fp32
    wcss of every iteration (evaluated in chunks on the GPU); iterations run,
    wcss and codebooks equal the oracle's bit for bit."""
    w = synth.WORKLOADS["corpus-1.52m"]
    x = corpus
    init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
    got = pq.train(x, w.dim, 0, m=w.m, ksub=w.ksub, max_iters=6, tol=1e-4, init_codebooks=init)
    ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=6, tol=1e-4, n_threads=16)
    assert ref.status == 0
    assert np.array_equal(got.stats.iters_run, ref.iters_run)
    assert np.array_equal(_bits(got.stats.wcss), _bits(ref.wcss))
    assert np.array_equal(_bits(got.codebooks), _bits(ref.codebooks))


def _ulps(a, b):
    """|a - b| in units in the last place, per float (same-sign finite floats)."""
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.fixture(scope="module")
def paper_60m_device():
    """The 60M-vector training sample as the benchmark makes it: generated on
    the device by the kernel form of the generator, with the seeded-shuffle
    codebooks read from those device rows.  Yields (workload, device rows,
    host copy of the same bytes, init codebooks)."""
    w = synth.WORKLOADS["paper-60m"]
    t0 = time.perf_counter()
    gen = synth.DeviceCorpus(w)
    dx = device.DeviceArray((w.n, w.dim), np.float32)
    gen.fill(dx, w.n)
    init = gen.shuffle_init(dx, w.n, w.m, w.ksub, w.seed)
    x = dx.to_host()
    gen.free()
    _log(f"paper-60m: generated {w.n:,} x {w.dim} on the device and copied back in "
         f"{time.perf_counter() - t0:.1f} s")
    yield w, dx, x, init
    dx.free()


@pytest.mark.timeout(300)
def test_device_generator_matches_host_generator(gpu, paper_60m_device):
    """The device generator (synth_gpu.hip) and the host one (synth.c) draw
    the same rows from the same counters; the device's double-precision
    log / sqrt / sincos may differ from glibc's in the last bit, so a float
    may differ by one unit in the last place.  On a 1,000,000-row slice of
    the 60M sample, every float is within 1 ulp and the differing ones are
    counted.  (Every oracle comparison of the 60M and 200M workloads feeds
    the oracle the device-generated bytes themselves.)"""
    w, _, x, _ = paper_60m_device
    first, rows = 30_000_000, 1_000_000
    host = synth.residuals(w, rows, first=first)
    dev = x[first:first + rows]
    same_sign = np.signbit(host) == np.signbit(dev)
    near_zero = (np.abs(host) < 1e-30) & (np.abs(dev) < 1e-30)
    assert np.all(same_sign | near_zero)
    u = _ulps(host.reshape(-1), dev.reshape(-1))
    n_diff = int(np.count_nonzero(u))
    _log(f"device vs host generator: {n_diff} of {u.size} floats differ, max {int(u.max())} ulp")
    assert int(u.max()) <= 1


@pytest.mark.timeout(300)
def test_paper_scale_60m_two_iterations_vs_oracle(gpu, paper_60m_device):
    """The benchmark's 60M training run (device-generated rows, seeded-shuffle
    init, m16 k256) for its first 2 Lloyd iterations, against the oracle on
    column slices: subspaces are trained independently
    (src/index/pq.zig:200-205), so columns 0-7 trained as m=2 from the first
    two init codebooks are subspaces 0-1 of the full run, and columns 56-63
    are subspaces 14-15 (the second training stream's half).  Both
    iterations' codebooks of those four subspaces are compared bit for bit;
    their largest clusters hold about 1.4M members."""
    w, dx, x, init = paper_60m_device
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    t0 = time.perf_counter()
    stats = device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, 2, NEVER, trace=True)
    device.synchronize()
    _log(f"paper-60m: 2 traced iterations on the GPU in {time.perf_counter() - t0:.2f} s")
    dinit.free()
    dcb.free()
    D = w.dsub
    for lo in (0, 14):
        xs = np.ascontiguousarray(x[:, lo * D:(lo + 2) * D])
        t0 = time.perf_counter()
        ref = orc.pq_train(xs, 2 * D, 2, w.ksub, init=init[lo:lo + 2], max_iters=2, tol=NEVER,
                           n_threads=16, trace=True)
        _log(f"paper-60m: oracle on subspaces {lo}-{lo + 1} in {time.perf_counter() - t0:.1f} s")
        assert ref.status == 0
        for t in range(2):
            got = stats[3][t][lo:lo + 2]
            diff = np.count_nonzero(_bits(got) != _bits(ref.trace[t]))
            assert diff == 0, f"iteration {t}, subspaces {lo}-{lo + 1}: {diff} floats differ"
        del xs


@pytest.mark.timeout(300)
def test_paper_scale_60m_resident(gpu, paper_60m_device):
    """60,000,000 x 64 residuals resident in HBM (the benchmark's
    device-generated rows), m16 k256, 25 iterations, through properties
    that hold at any size."""
    w, dx, x, init = paper_60m_device
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((w.n, w.m), np.uint8)

    def train(iters):
        t = time.perf_counter()
        it, wc, _ = device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, iters, NEVER,
                                        stats=True)
        device.synchronize()
        _log(f"paper-60m: {iters} iterations in {time.perf_counter() - t:.2f} s")
        assert np.all(it == iters)
        return wc.astype(np.float64), dcb.to_host()

    wcss1, _ = train(1)
    wcss5, _ = train(5)
    _, cb24 = train(w.iters - 1)
    device.encode_device(dx, w.n, w.dim, w.m, w.ksub, dcb, dcodes)
    codes24 = dcodes.to_host()
    wcss25, cb25 = train(w.iters)
    for a in (dinit, dcb, dcodes):
        a.free()

    # WCSS of Lloyd iterations does not increase (src/tac/kmeans.zig:503-521)
    assert np.all(wcss5 <= wcss1) and np.all(wcss25 <= wcss5)

    # encode with cb24 = the final iteration's assignment; oracle on a sample
    sample = slice(17, None, 6007)
    assert np.array_equal(codes24[sample], orc.pq_encode(x[sample], w.dim, w.m, w.ksub, cb24,
                                                         n_threads=16))

    # every non-empty cluster of the last update is the serial mean of its points
    D = w.dsub
    checked = 0
    for m in (0, 9, 15):
        cm = codes24[:, m]
        counts = np.bincount(cm, minlength=w.ksub)
        for c in (int(np.argmax(counts)), int(np.argmin(np.where(counts, counts, 1 << 40))), 77):
            if counts[c] == 0:
                continue
            pts = x[cm == c, m * D:(m + 1) * D]
            assert np.array_equal(_bits(cb25[m, c]), _bits(_serial_mean(pts))), (m, c)
            checked += 1
    assert checked >= 6

    # training the same state further is deterministic
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    _, again = train(w.iters)
    dinit.free()
    dcb.free()
    assert np.array_equal(_bits(again), _bits(cb25))


@pytest.mark.timeout(300)
def test_stream_encode_200m(gpu):
    """200,000,000 residuals in 10M-vector chunks generated on the device, as
    the benchmark streams them, encoded against fixed N(0, 0.05^2) codebooks:
    every chunk's codes equal the oracle's on the device-generated bytes, in
    full for the first and last chunks and on a sample of the others, and
    the codes of the whole stream account for every vector."""
    w = synth.WORKLOADS["stream-200m"]
    chunk = 10_000_000
    gen = synth.DeviceCorpus(w)
    cb = synth.gauss_codebooks(w.seed, w.m, w.ksub, w.dsub, 0.05)
    dcb = device.DeviceArray.from_host(cb)
    dx = device.DeviceArray((chunk, w.dim), np.float32)
    dcodes = device.DeviceArray((chunk, w.m), np.uint8)
    hist = np.zeros((w.m, w.ksub), np.int64)
    t_enc = 0.0
    last = w.n - chunk
    for first in range(0, w.n, chunk):
        gen.fill(dx, chunk, first)
        t0 = time.perf_counter()
        device.encode_device(dx, chunk, w.dim, w.m, w.ksub, dcb, dcodes)
        device.synchronize()
        t_enc += time.perf_counter() - t0
        codes = dcodes.to_host()
        x = dx.to_host()
        for m in range(w.m):
            hist[m] += np.bincount(codes[:, m], minlength=w.ksub)
        s = slice(None) if first in (0, last) else slice(first % 997, None, 20011)
        assert np.array_equal(codes[s], orc.pq_encode(x[s], w.dim, w.m, w.ksub, cb,
                                                      n_threads=16)), first
        _log(f"stream-200m: chunk at {first:,} checked")
    for a in (dcb, dx, dcodes):
        a.free()
    gen.free()
    _log(f"stream-200m: {w.n:,} vectors, encode {t_enc:.2f} s ({w.n / t_enc / 1e6:.0f} Mvec/s)")
    assert np.all(hist.sum(axis=1) == w.n)
