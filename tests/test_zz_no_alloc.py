"""tac_pq_encode_device_noalloc (the encode that allocates no device memory)
against tac_pq_encode_device on the same inputs, byte for byte, over two
calls in a row with the second on fewer rows: the static scratch keeps the
first call's contents, so the second call must not depend on them."""
import numpy as np
import pytest

from tac_gpu import device, errors, lib, synth

pytestmark = pytest.mark.gpu


def _encode(fn, dx, n, dim, m, ksub, dcb, fill):
    """Codes of the first n rows; the output starts filled with `fill`, so a
    row one entry point leaves unwritten differs from the other's."""
    dt = device.code_dtype(ksub)
    out = device.DeviceArray.from_host(np.full((n, m), fill, dt))
    errors.check(fn(dx.ptr, n, dim, m, ksub, dcb.ptr, out.ptr, None))
    device.synchronize()
    codes = out.to_host()
    out.free()
    return codes


# (m, ksub, rows of the first call, rows of the second call).  At m16 the
# scratch holds batches of 245,760 rows: the first call runs two full
# batches and a 5,000-row tail (full search); m64 batches are 49,152 rows; m8
# (dsub 8) takes the matrix-core screen in batches of 1,046,528 rows; ksub
# 1024 and calls under 16,384 rows take the full search throughout.
CASES = [
    (16, 256, 2 * 245_760 + 5_000, 40_000),
    (64, 256, 300_000, 20_000),
    (8, 256, 1_100_000, 17_000),
    (32, 256, 70_000, 12_000),
    (16, 1024, 60_000, 9_000),
    (16, 3, 30_000, 16_384),
]


@pytest.mark.parametrize("m,ksub,n1,n2", CASES)
def test_noalloc_encode_matches_encode_device(gpu, m, ksub, n1, n2):
    w = synth.WORKLOADS["paper-60m"]
    dim = w.dim
    print(f"[no-alloc] m={m} ksub={ksub} n={n1},{n2}", flush=True)
    x = synth.residuals(w, n1, first=12_345)
    cb = synth.shuffle_init(x, m, ksub, 5)  # codewords are data points
    dx = device.DeviceArray.from_host(x)
    dcb = device.DeviceArray.from_host(cb)
    try:
        refs = [_encode(lib.tac_pq_encode_device, dx, n, dim, m, ksub, dcb, 0) for n in (n1, n2)]
        got = [_encode(lib.tac_pq_encode_device_noalloc, dx, n, dim, m, ksub, dcb, 0xFF)
               for n in (n1, n2)]
    finally:
        dx.free()
        dcb.free()
    for r, g, n in zip(refs, got, (n1, n2)):
        diff = int(np.count_nonzero(r != g))
        assert diff == 0, f"{n} rows: {diff} codes differ"
