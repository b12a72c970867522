"""The wave broadcast the ring workers use (rl_wave_bcast_u32 / _u64) through
rl_hip_wave_broadcast_selftest, in the shape of the reference's warp
broadcast test (test/test_bench.cu:623-656): every lane of each wave receives
the source lane's 64-bit sequence id, 32-bit offset and 64-bit cookie; the
second wave broadcasts from lane 37, not 0."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_wave_broadcast_u32_u64(rl, gpu):
    L = rl.lib()
    seq, off, cookie = rl.DeviceBuffer(128 * 8, zero=True), rl.DeviceBuffer(128 * 4, zero=True), \
        rl.DeviceBuffer(128 * 8, zero=True)
    print("[broadcast] two waves, sources lane 0 and lane 37", flush=True)
    rl.check(L.rl_hip_wave_broadcast_selftest(seq.ptr, off.ptr, cookie.ptr), "rl_hip_wave_broadcast_selftest")
    s, o, c = seq.download(np.uint64, 128), off.download(np.uint32, 128), cookie.download(np.uint64, 128)
    for w in range(2):
        assert np.all(s[64 * w:64 * w + 64] == np.uint64(0x123456789ABCDEF0 + w)), w
        assert np.all(o[64 * w:64 * w + 64] == np.uint32(77 + w)), w
        assert np.all(c[64 * w:64 * w + 64] == np.uint64(0x0FEDCBA987654321 ^ w)), w
    for b in (seq, off, cookie):
        b.close()


def test_wave_broadcast_refuses_null(rl, gpu):
    assert rl.lib().rl_hip_wave_broadcast_selftest(None, None, None) == -1
    assert "NULL" in rl._err()
