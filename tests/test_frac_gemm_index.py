"""The half-integer-rate GEMM's decode indexing on the CPU (gemm_ws_kernel's
FR > 0 branch and gw_decode_frac / chunk_cw_frac in
plugins_amd/csrc/exl3_kern.h, restated with numpy): every thread's dword
offsets stay inside its tile, and the codewords its windows extract are the
tile's codewords as the oracle unpacks them (sushi_ds41/src/sushi/exl3/
expert_exl3.zig:317-336, pinned by the bit-by-bit definition), at n = 24 and
40 (turboexl3_ds41/src/bank/frac.zig:42-44).  Runs before the kernel does."""
import numpy as np
import pytest

from oracle import oracle as O


def words_u32(hw):
    # u32 word m = hw[2m] | hw[2m+1] << 16 (expert_exl3.zig:313-315)
    hw = hw.astype(np.uint32)
    return hw[0::2] | (hw[1::2] << 16)


def alignbit(hi, lo, s):
    return int(((int(hi) << 32 | int(lo)) >> s) & 0xFFFFFFFF)


def ubfe(v, off, width):
    return (int(v) >> off) & ((1 << width) - 1)


def thread_codewords(tile_words, FR, c):
    """Codewords 32c .. 32c+31 as the kernel's thread of chunk c forms them."""
    n = 8 * FR
    NW = 4 * FR
    NB = (FR + 1) // 2
    LW = NB + 1
    hs = (c * FR - 1 + n) % n
    low = hs & 1
    b0 = (hs >> 1) - (0 if low else 1)
    off = [(b0 + j) % NW for j in range(LW)]
    assert all(0 <= o < NW for o in off)
    sh = 16 if low else 0
    wn = [tile_words[o] for o in off]
    wd = [alignbit(wn[j], wn[j + 1], sh) for j in range(NB)]
    out = []
    for i in range(32):
        E = 16 + ((i + 1) * FR) // 2
        J0, J1 = (E - 16) >> 5, (E - 1) >> 5
        assert J1 < NB
        if J0 == J1:
            out.append(ubfe(wd[J0], 31 - ((E - 1) & 31), 16))
        else:
            out.append(alignbit(wd[J0], wd[J1], 31 - ((E - 1) & 31)) & 0xFFFF)
    return out


@pytest.mark.parametrize("FR", [3, 5])
def test_frac_threads_extract_the_tiles_codewords(FR):
    n = 8 * FR
    rng = np.random.default_rng(FR)
    for _ in range(20):
        hw = rng.integers(0, 65536, n, dtype=np.uint16)
        want = O.unpack_tile(hw, n, bitwise=True)
        tw = words_u32(hw)
        got = [cw for c in range(8) for cw in thread_codewords(tw, FR, c)]
        np.testing.assert_array_equal(np.array(got, np.uint16), want)


def test_frac_index_math_catches_a_missing_wrap():
    # planted on the CPU: chunk 0's history read from dword 0 instead of the
    # tile's last halfword fails the bit-by-bit definition
    FR, n = 3, 24
    hw = np.random.default_rng(9).integers(0, 65536, n, dtype=np.uint16)
    tw = words_u32(hw)
    want = O.unpack_tile(hw, n, bitwise=True)
    bad = list(tw)
    bad[n // 2 - 1] = (bad[n // 2 - 1] ^ 0xFFFF) & 0xFFFFFFFF  # only the history halfword changes
    got0 = thread_codewords(bad, FR, 0)
    assert (np.array(got0, np.uint16) != want[:32]).any()
