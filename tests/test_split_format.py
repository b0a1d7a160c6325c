"""Host-side tables of the split device format (huffman_codebook.
split_tables): a CPU packer and a CPU restatement of the GPU decode step
(window of 30 bits at q - 2, 14-bit two-code table index, shift by the two
code lengths) recover every weight bit for bit, codes stay within 7 bits,
and the code is a complete prefix code over the high bytes that occur."""
import numpy as np
import pytest

import huffman_codebook as hc


def bf16_codebook(rng, n, scale=0.02):
    w = rng.standard_normal(4 * n).astype(np.float32) * np.float32(scale)
    b = (w.view(np.uint32) >> 16) << 16
    u = np.unique(b)[:n]
    return u.view(np.float32)


def cpu_pack(idx, sym_code, sym_raw):
    """Column layout exactly as cbq_split_pack writes it."""
    n = idx.size
    n_sub, n_chunks = n // 64, n // 4096
    code, ln = sym_code & 0xFFFFFF, sym_code >> 24
    sub_bits = ln[idx].reshape(n_sub, 64).sum(1)
    rows = np.maximum((sub_bits.reshape(n_chunks, 64).max(1) + 31) // 32, 1)
    row_off = np.concatenate([[0], np.cumsum(rows)]).astype(np.int64)
    cw = np.zeros((row_off[-1], 64), np.uint32)
    for s in range(n_sub):
        c, l = divmod(s, 64)
        acc, nb, r = 0, 0, 0
        for v in idx[s * 64:(s + 1) * 64]:
            acc |= int(code[v]) << nb
            nb += int(ln[v])
        for r in range(rows[c]):
            cw[row_off[c] + r, l] = (acc >> (32 * r)) & 0xFFFFFFFF
    return cw, row_off, sym_raw[idx]


def cpu_decode(cw, row_off, raw, lut, n):
    """The kernel's decode walk, restated on the CPU: float32 bits per weight.
    Per group of 4 weights one 30-bit window (alignbit at q - 2), then two
    table reads, each giving two high bytes and their total code length."""
    out = np.zeros(n, np.uint32)
    for s in range(n // 64):
        c, l = divmod(s, 64)
        col = cw[row_off[c]:row_off[c + 1], l].astype(np.uint64)
        stream = 0
        for r, wd in enumerate(col):
            stream |= int(wd) << (32 * r)
        stream <<= 2                                   # bit q of the stream at bit q + 2
        q = 0
        for g in range(16):
            w = (stream >> q) & 0xFFFFFFFF             # alignbit(hi, lo, q - 2)
            for u in range(0, 4, 2):
                e = int(lut[(w & 0xFFFC) >> 2])
                for k, hb in ((0, e >> 24), (1, (e >> 16) & 0xFF)):
                    i = s * 64 + 4 * g + u + k
                    out[i] = (hb << 24) | (int(raw[i]) << 16)
                w >>= (e & 31)
                q += e & 0xFF
    return out


@pytest.mark.parametrize("seed,C,skew", [(0, 300, 1.0), (1, 4000, 1.3), (2, 40, 0.0), (3, 5, 2.0)])
def test_split_roundtrip(seed, C, skew):
    rng = np.random.default_rng(seed)
    cb = bf16_codebook(rng, C)
    C = cb.size
    p = 1.0 / np.arange(1, C + 3) ** skew             # alphabet C+2: indices past C clamp
    p /= p.sum()
    idx = rng.choice(C + 2, size=2 * 4096, p=p).astype(np.int64)
    counts = np.bincount(idx, minlength=C + 2)
    sym_code, sym_raw, lut = hc.split_tables(cb, counts)
    assert int((sym_code >> 24).max()) <= hc.SPLIT_MAX_LEN
    cw, row_off, raw = cpu_pack(idx, sym_code, sym_raw)
    assert int(np.diff(row_off).max()) <= 14
    got = cpu_decode(cw, row_off, raw, lut, idx.size)
    want = cb[np.minimum(idx, C - 1)].view(np.uint32)
    assert np.array_equal(got, want)


def test_split_code_is_complete_prefix_code():
    rng = np.random.default_rng(7)
    cb = bf16_codebook(rng, 2000)
    counts = rng.integers(0, 50, cb.size)
    sym_code, _, lut = hc.split_tables(cb, counts)
    his = cb.view(np.uint32) >> 24
    used = np.unique(his[counts > 0])
    lens = {int(h): int(sym_code[np.nonzero(his == h)[0][0]] >> 24) for h in used}
    assert sum(2.0 ** -L for L in lens.values()) == pytest.approx(1.0)
    # every table entry names two used high bytes and their total code length
    assert set(int(v) >> 24 for v in lut) == set(int(h) for h in used)
    for v in lut[::97]:
        h1, h2 = int(v) >> 24, (int(v) >> 16) & 0xFF
        assert lens[h1] + lens[h2] == int(v) & 0xFF


def test_split_rejects_non_bf16_and_too_many_high_bytes():
    cb = np.array([0.5, 0.1], np.float32)              # 0.1 is not a bf16 number
    assert hc.split_tables(cb, [3, 4]) is None
    e = np.arange(1, 140, dtype=np.uint32) << 24        # 139 distinct high bytes
    assert hc.split_tables(e.view(np.float32), np.ones(139)) is None


def test_split_single_exponent():
    cb = (np.array([0x3F80, 0x3F81, 0xBF80], np.uint32) << 16).view(np.float32)   # 1.0, ~1.0, -1.0
    idx = np.tile(np.array([0, 1, 2, 1]), 1024)
    sym_code, sym_raw, lut = hc.split_tables(cb, np.bincount(idx))
    assert set(int(x) >> 24 for x in sym_code) == {1}
    cw, row_off, raw = cpu_pack(idx, sym_code, sym_raw)
    assert np.array_equal(cpu_decode(cw, row_off, raw, lut, idx.size), cb[idx].view(np.uint32))
