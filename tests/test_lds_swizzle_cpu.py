"""LDS tile swizzle (swz<KCH> in flash-attention-turing_amd/csrc/fa_common.h)
against the read patterns of TileReader, on 64 four-byte banks: a
ds_read_b128 serves 16 lanes per cycle, a ds_read_b64 32, and a phase is
conflict-free when its lanes touch every bank once.  The MFMA A-operand read
(row sigma(lane % 32), chunk 2g + lane / 32) and the transposed read
(ds_read_b64_tr_b16: rows 8h + j (+4), 8 bytes of chunk x) must both be
conflict-free at head_dim 64 and 128, for every row offset the kernels use.
The same model reads 2-way conflicts for the head_dim 64 mask used before,
as the PMC counter SQ_LDS_BANK_CONFLICT did."""

import pytest


def sigma(i):
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1)


def swz(kch, row):
    if kch == 16:
        return (4 if row & 1 else 0) ^ (10 if row & 2 else 0) ^ (2 if row & 4 else 0) ^ (1 if row & 8 else 0)
    return (4 if row & 2 else 0) ^ (1 if row & 4 else 0) ^ (2 if row & 8 else 0)


def old_swz64(row):
    return (2 if row & 1 else 0) ^ (4 if row & 2 else 0) ^ (1 if row & 8 else 0)


def excess(phases, width):
    """Extra bank cycles over all phases (0 = conflict-free)."""
    total = 0
    for lanes in phases:
        count = {}
        for addr in lanes:
            for w in range(width // 4):
                bank = (addr // 4 + w) % 64
                count[bank] = count.get(bank, 0) + 1
        total += max(count.values()) - 1
    return total


def a_operand_excess(hd, f, r0):
    kch, rowb = hd // 8, hd * 2
    total = 0
    for g in range(hd // 16):
        addrs = []
        for lane in range(64):
            row = sigma(lane & 31)
            chunk = (lane >> 5) + 2 * g
            addrs.append((r0 + row) * rowb + (((chunk ^ f(r0 + row)) & (kch - 1)) << 4))
        total += excess([addrs[i:i + 16] for i in range(0, 64, 16)], 16)
    return total


def tr_operand_excess(hd, f, r0):
    kch, rowb = hd // 8, hd * 2
    total = 0
    for dt in range(hd // 32):
        for hs in range(2):
            addrs = []
            for lane in range(64):
                j, q, db, h = (lane & 15) >> 2, lane & 3, (lane >> 4) & 1, lane >> 5
                x, byte = 2 * db + (q >> 1), (q & 1) * 8
                r = 8 * h + j + 4 * hs
                addrs.append((r0 + r) * rowb + ((((x + 4 * dt) ^ f(r0 + r)) & (kch - 1)) << 4) + byte)
            total += excess([addrs[:32], addrs[32:]], 8)
    return total


@pytest.mark.parametrize("hd", [64, 128])
def test_both_read_forms_conflict_free(hd):
    f = lambda r: swz(hd // 8, r)  # noqa: E731
    for r0 in (0, 32, 64, 96):  # A operands start at multiples of 32 rows
        assert a_operand_excess(hd, f, r0) == 0
    for r0 in range(0, 128, 16):  # transposed operands at multiples of 16
        assert tr_operand_excess(hd, f, r0) == 0


def test_swizzle_repeats_every_16_rows():
    """TileCopier relies on copies 16k rows apart sharing the swizzle."""
    for kch in (8, 16):
        assert all(swz(kch, r) == swz(kch, r + 16) for r in range(64))


def test_model_sees_the_old_head_dim_64_conflicts():
    assert a_operand_excess(64, old_swz64, 0) > 0


def reader_bases(hd, lane):
    """TileReader<hd>::init: the lane's A-operand base and its two transposed-read bases."""
    kch, rowb = hd // 8, hd * 2
    col, h = lane & 31, lane >> 5
    row = sigma(col)
    a_base = row * rowb + (((h ^ swz(kch, row)) & (kch - 1)) << 4)
    j, q, db = (lane & 15) >> 2, lane & 3, (lane >> 4) & 1
    x, byte = 2 * db + (q >> 1), (q & 1) * 8
    tr = [(8 * h + j + 4 * hs) * rowb + (((x ^ swz(kch, 8 * h + j + 4 * hs)) & (kch - 1)) << 4) + byte
          for hs in range(2)]
    return a_base, tr


def tile_offsets(hd):
    """Every tile offset the kernels add to a lane base once (a_operand_at / tr_operand_at):
    the dK/dV stages and the wave's V rows, the dQ and forward stages."""
    dkv_qtile = 32 * hd * 2
    dkv_stage = 2 * dkv_qtile + 2 * 64 * 4
    offs = {0, dkv_stage} | {2 * dkv_stage + kg * 32 * hd * 2 for kg in range(4)}
    kv_stage = 2 * (64 * hd * 2)  # dQ and forward: a K and a V tile of 64 keys
    return offs | {kv_stage}


@pytest.mark.parametrize("hd", [64, 128])
def test_tile_offset_commutes_with_step_xor(hd):
    """The kernels form base + t once per tile and read at (base + t) ^ m for the step mask
    m (g << 5, dt << 6); that address must be the per-read form (base ^ m) + t, for every
    lane base, tile offset and step."""
    masks = [g << 5 for g in range(hd // 16)] + [dt << 6 for dt in range(hd // 32)]
    for t in tile_offsets(hd):
        assert t % 512 == 0
        for lane in range(64):
            a_base, tr = reader_bases(hd, lane)
            for base in (a_base, *tr):
                for m in masks:
                    assert (base + t) ^ m == (base ^ m) + t


def test_commuting_needs_the_offset_alignment():
    """The identity needs the offset's bits up to the highest step bit (bit 7) clear; 512 is
    what the kernels assert.  A plausible slip, an offset inside a row (here two 16-byte
    chunks), breaks it for some lane and step, so the check above can fail."""
    assert any((base + 32) ^ (g << 5) != (base ^ (g << 5)) + 32
               for lane in range(64) for base in (reader_bases(128, lane)[0],) for g in range(8))
