"""The dS tile layout shared by the dK / dV kernel (writer) and the dQ kernel
(reader), simulated on the CPU (tilelang-fa-v100_amd/csrc/fa_bwd_mfma.h,
fa_bwd_ds.h).

Writer: lane (key lr, half lh) of a dK / dV wave holds, as its B-operand chunk
kq, dS of query rows 16kq + 8(x/4) + 4lh + x%4 (x = 0..7, the MFMA
accumulator layout); it stores the chunk as 16-byte row
16(2(lr/16) + (lr/8)%2) + 8lh + 4(((lr/4)%2) ^ kq) + lr%4 of 1 KB block kq.
Reader: ds_read_b64_tr_b16 gives lane 16g + i, element j, element i%4 of the
8 bytes addressed by lane 16g + 4j + i/4; the dQ kernel's lane l must receive
dS[query l%32][key 16kc + 8(l/32) + 4r + j] (read r, key chunk kc) so that it
pairs with the A operand Kᵀ read the same way.  A mistake in either index
formula (a swapped half, a wrong XOR) breaks the element check; a layout
that is right but slow breaks the bank-group check.
"""


def _writer_layout():
    mem = {}
    for lr in range(32):
        for lh in range(2):
            prow = 16 * (2 * (lr >> 4) + ((lr >> 3) & 1)) + 8 * lh + (lr & 3)
            g1 = (lr >> 2) & 1
            for kq in range(2):
                row = prow + 4 * (g1 ^ kq)
                for x in range(8):
                    q = 16 * kq + 8 * (x // 4) + 4 * lh + x % 4
                    off = kq * 1024 + 16 * row + 2 * x
                    assert off not in mem, "two elements stored at one address"
                    mem[off] = (q, lr)
    return mem


def _reader_offset(s, r):
    lh, kq = s >> 5, (s >> 4) & 1
    return (1024 * kq + 16 * (16 * lh + 8 * (s & 1) + 4 * (r ^ kq) + ((s & 15) >> 2)) +
            8 * ((s & 3) >> 1))


def test_writer_fills_the_tile_once():
    mem = _writer_layout()
    assert sorted(mem) == list(range(0, 2048, 2))
    assert sorted(set(mem.values())) == [(q, k) for q in range(32) for k in range(32)]


def test_reader_gets_the_mfma_operand():
    mem = _writer_layout()
    for kc in range(2):
        for r in range(2):
            for lane in range(64):
                g, i = lane // 16, lane % 16
                for j in range(4):
                    src = 16 * g + 4 * j + i // 4
                    q, key = mem[_reader_offset(src, r) + 512 * kc + 2 * (i % 4)]
                    assert q == lane % 32
                    assert key == 16 * kc + 8 * (lane // 32) + 4 * r + j


def test_reader_is_free_of_bank_conflicts():
    # 64 banks of 4 bytes: the 32 lanes of a half wave read 8 bytes each and
    # must cover 32 distinct 8-byte bank pairs.
    for kc in range(2):
        for r in range(2):
            for half in range(2):
                pairs = {((_reader_offset(s, r) + 512 * kc) % 256) // 8
                         for s in range(32 * half, 32 * half + 32)}
                assert len(pairs) == 32


def test_each_store_writes_one_whole_block():
    # A store instruction of the writer (fixed kq) covers its 1 KB block.
    for kq in range(2):
        rows = set()
        for lr in range(32):
            for lh in range(2):
                prow = 16 * (2 * (lr >> 4) + ((lr >> 3) & 1)) + 8 * lh + (lr & 3)
                rows.add(prow + 4 * (((lr >> 2) & 1) ^ kq))
        assert rows == set(range(64))
