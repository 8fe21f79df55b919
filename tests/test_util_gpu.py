"""GPU checks of the bit-exact dequant (p0_q4_dequant) and the synthetic-data fillers, against the oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,w_off", [(128, 256, 0), (192, 96, 4), (64, 2048, 16)])
def test_dequant_bit_exact(dev, N, K, w_off):
    """fl32(q s + m) and its fp16 tile value, bit for bit (engine/kcheck.js:32, engine/ops/gemm.js:147-148)"""
    W = O.randn(N * K, 5 + N, 0.05)
    W[:K] *= 1e4                      # a row with large values next to tiny ones: wide exponent spreads in one tile
    b, deq = O.pack_q4(W, N, K)
    buf = np.zeros(w_off + b.nbytes, np.uint8)
    buf[w_off:] = b
    wb = capi.to_device(buf)
    o32 = capi.Buffer(N * K * 4).fill_u32(0x7FC00000)
    o16 = capi.Buffer(N * K * 2).fill_u32(0x7E007E00)
    capi.q4_dequant(wb, N, K, out32=o32, out16=o16, w_off=w_off)
    g32, g16 = o32.read(np.uint32), o16.read(np.uint16)
    w32, w16 = O.dequant_q4(b, N, K)
    assert np.array_equal(g32, w32.view(np.uint32).ravel())
    assert np.array_equal(g32, deq.view(np.uint32).ravel())
    assert np.array_equal(g16, w16.ravel())
    for x in (wb, o32, o16):
        x.free()


def test_fill_q4_sym_matches_oracle(dev):
    N, K = 256, 512
    wb = capi.Buffer(N // 64 * K // 32 * 1280)
    capi.fill_q4_sym(wb, N, K, 1234, 0.02)
    got = wb.read(np.uint8).reshape(-1, 1280)
    want = O.fill_q4_sym(N, K, 1234, 0.02).reshape(-1, 1280)
    assert np.array_equal(got[:, :1024], want[:, :1024])                 # code words: integer hash, exact
    gs = got[:, 1024:].copy().view(np.uint32).ravel()
    ws = want[:, 1024:].copy().view(np.uint32).ravel()
    mismatch = np.count_nonzero(gs != ws)
    # scales go through float64 log / cos on both sides: libm last-ulp differences may move a rare fp16 rounding
    assert mismatch <= max(1, gs.size // 10000), mismatch
    wb.free()


def test_fill_randn_matches_oracle(dev):
    n = 100_000
    b32, b16 = capi.Buffer(n * 4), capi.Buffer(n * 2)
    capi.fill_randn(b32, n, 77)
    capi.fill_randn(b16, n, 77, as_f16=True)
    w32, w16 = O.fill_randn(n, 77)
    g32, g16 = b32.read(np.float32), b16.read(np.uint16)
    assert np.count_nonzero(g16 != w16) <= 10
    assert np.array_equal(g32.view(np.uint32) == w32.view(np.uint32), g16 == w16)
    b32.free(); b16.free()


@pytest.mark.parametrize("src_off,dst_off,n", [(0, 0, 1 << 20), (4, 12, 4096 + 8), (16, 32, 12)])
def test_copy(dev, src_off, dst_off, n):
    """runner.copy (engine/core/gpu.js:237-242): the 16-byte path when everything is 16-aligned, else 4-byte words"""
    src = np.random.default_rng(5).integers(0, 2**32, (src_off + n) // 4, dtype=np.uint32)
    a = capi.to_device(src)
    b = capi.Buffer(dst_off + n + 64).fill_u32(0xDEADBEEF)
    capi.copy(a, src_off, b, dst_off, n)
    got = b.read(np.uint32)
    assert np.array_equal(got[dst_off // 4: (dst_off + n) // 4], src[src_off // 4:])
    assert np.all(got[: dst_off // 4] == 0xDEADBEEF) and np.all(got[(dst_off + n) // 4:] == 0xDEADBEEF)
    a.free()
    b.free()


def test_copy_errors(dev):
    a = capi.Buffer(256)
    with pytest.raises(capi.P0Error, match="multiples of 4"):
        capi.copy(a, 2, a, 128, 16)
    with pytest.raises(capi.P0Error, match="overlap"):
        capi.copy(a, 0, a, 16, 64)
    a.free()


def test_probe_mfma_counts_its_flops(dev):
    """the matrix-core probe (p0_probe_mfma) enqueues 8 waves x 4 chains x iters 32x32x16 MFMAs per CU, reports that
    many flops, and leaves its sink alone (its sums never take the sentinel value)"""
    cus = capi.device_info()["cu_count"]
    sink = capi.Buffer(4 * cus + 16).fill_u32(0x12345678)
    fl = capi.probe_mfma(100, sink)
    capi.done()
    assert fl == cus * 8 * 4 * 32 * 32 * 16 * 2 * 100
    assert np.all(sink.read(np.uint32) == 0x12345678)
    with pytest.raises(capi.P0Error, match="probe_mfma"):
        capi.probe_mfma(0, sink)
    sink.free()


def test_probe_read_reads_the_whole_buffer(dev):
    """the read probe (p0_probe_read) folds every 16-byte piece it loads: a buffer whose only nonzero word sits in the
    last piece (the grid-stride loop's last iterations) folds to the sentinel and writes the sink; a zero buffer
    leaves it alone; sizes that are not multiples of 16 are refused"""
    n = 64 << 20
    buf = capi.Buffer(n).fill_u32(0)
    sink = capi.Buffer(16).fill_u32(0x12345678)
    capi.probe_read(buf, n, sink)
    capi.done()
    assert sink.read(np.uint32)[0] == 0x12345678
    buf.upload(np.array([0x9E3779B9, 0, 0, 0], np.uint32), off=n - 16)
    capi.probe_read(buf, n, sink)
    capi.done()
    assert sink.read(np.uint32)[0] == 0x9E3779B9
    with pytest.raises(capi.P0Error, match="probe_read"):
        capi.probe_read(buf, n - 8, sink)
    buf.free()
    sink.free()
