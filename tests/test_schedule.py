"""CPU replica of the balanced split-K schedule's integer arithmetic, fuzzed.

``paged_attention_balanced_kernel`` (decodekernels_amd/csrc/paged_attention.hip)
lays the (sequence, KV head) streams end to end on a line of cost positions --
a stream costs its 16-token tiles plus a fixed per-stream overhead -- and
gives workgroup w the positions [first_pos(w), first_pos(w + 1)), the first
half of the grid ``pair_ratio / 100`` times the share of the second half. Each
piece (one stream's tiles inside one share) writes workspace row
``w - owner(first tile)`` of its stream, and the workgroup holding a stream's
last tile marks the row after its own empty when there is one. The reduce
merges the rows before the first empty one. The kernel evaluates ``owner``
once, for the stream that holds the share's first position: every later
stream it enters starts inside the share, so its row is 0 (checked here
against ``w - owner(first tile)`` for every piece). Share boundaries are kept
in 32-bit integers (checked below 2^31).

This file restates that arithmetic line for line and checks, over the
benchmark configurations and random shapes (lengths, heads, partitions, grid
sizes, pair ratios, stream costs, block sizes), the invariants the kernel and
the reduce rely on:

* every tile of every stream is processed exactly once, in order;
* a stream's pieces use rows 0 .. n-1, n <= max_partitions, and row n is
  marked empty whenever n < max_partitions (so the reduce reads exactly the
  pieces, however the workspace started);
* each sub-unit (at most 64 tiles) spans at most 64 cache blocks, the block-
  table entries one wave holds (one per lane) for block sizes that are
  multiples of 16;
* the 128K batch-1 configuration spans more than 64 rows per stream (the
  reduce's second ballot pass, also asserted on the GPU);
* when the work is too small for the pair ratio above the 64-tile minimum
  share, the second half of the grid keeps the minimum and still gets work
  (the ratio shrinks instead of the first half's shares taking it all).
"""

import math
import random

import pytest

TILE = 16
PART = 512
MIN_SHARE = 64


def balanced_schedule(lens, hkv, P, grid, pair_ratio, stream_cost, mistake=None, with_subs=True, lockstep=False):
    """Pieces {(seq, kv): [(group, row, tile_lo, tile_hi, sub_units)]} and
    marks {(seq, kv): row} as the kernel computes them for a launch of ``grid``
    workgroups. ``lockstep``: the line holds sequences only and groups of hkv
    consecutive workgroups share each share, one KV head each (else every
    workgroup is a group of one). ``mistake`` plants an error (tests show the
    checks catch it): "row" numbers rows from the owner of the stream's
    overhead instead of its first tile; "end" ends a piece one tile early;
    "clamp" keeps the pair ratio for small totals; "head" gives the lockstep
    walk the head of the group's first workgroup instead of its own."""
    S = len(lens)
    ln = [min(max(x, 0), P * PART) for x in lens]
    tiles_of = [(x + TILE - 1) // TILE for x in ln]
    cost_len = [t + stream_cost if x > 0 else 0 for t, x in zip(tiles_of, ln)]
    pre = [0]
    for c in cost_len:
        pre.append(pre[-1] + c)
    R = hkv if lockstep else 1  # workgroups per group
    hl = 1 if lockstep else hkv  # KV heads laid on the line per sequence
    total = pre[S] * hl
    G = grid // R  # groups
    H = G // 2
    r = pair_ratio
    denom = H * r + (G - H) * 100
    share_b = (total * 100 + denom - 1) // denom
    if share_b >= MIN_SHARE:
        share_a = max(MIN_SHARE, (share_b * r + 99) // 100)
    elif mistake == "clamp":  # the second half at the minimum, the ratio kept
        share_b = MIN_SHARE
        share_a = max(MIN_SHARE, (share_b * r + 99) // 100)
    else:  # too little work for the ratio above the minimum: the first half takes the rest
        share_b = MIN_SHARE
        share_a = max(MIN_SHARE, (total - (G - H) * MIN_SHARE + H - 1) // max(H, 1))
    split_at = H * share_a

    def first_pos(wg):
        return wg * share_a if wg < H else split_at + (wg - H) * share_b

    def owner(x):
        return x // share_a if x < split_at else H + (x - split_at) // share_b

    def cost_of(s):
        return pre[s + 1] - pre[s]

    assert max(split_at, first_pos(G)) < 2**31, "share boundaries must fit 32-bit integers"

    pieces, marks = {}, {}
    for x in range(grid):
        w = x // R
        kv0 = 0 if mistake == "head" else x - w * R
        if w >= G or first_pos(w) >= total:
            continue
        a = first_pos(w)
        b = min(first_pos(w + 1), total)
        lo, hi_s = 0, S
        while hi_s - lo > 1:
            mid = (lo + hi_s) >> 1
            if pre[mid] * hl <= a:
                lo = mid
            else:
                hi_s = mid
        st = {"seq": lo}
        assert cost_of(lo) > 0
        st["kv"] = kv0 + (a - pre[lo] * hl) // cost_of(lo)
        first0 = pre[lo] * hl + (st["kv"] - kv0) * cost_of(lo) + stream_cost
        anchor0 = first0 - stream_cost if mistake == "row" else first0
        first_row = w - owner(anchor0) if first0 < a else 0

        def advance():
            st["kv"] += 1
            if st["kv"] < kv0 + hl:
                return True
            st["kv"] = kv0
            while True:
                st["seq"] += 1
                if st["seq"] >= S:
                    return False
                if cost_of(st["seq"]) > 0:
                    return True

        def enter():
            while True:
                seq, kv = st["seq"], st["kv"]
                first = pre[seq] * hl + (kv - kv0) * cost_of(seq) + stream_cost
                n = tiles_of[seq]
                if first >= b:
                    return False
                t_lo = max(a, first) - first
                st["hi"] = min(b, first + n) - first - (1 if mistake == "end" else 0)
                if t_lo < st["hi"]:
                    row = first_row if first < a else 0
                    if mistake is None:
                        assert row == w - owner(first)
                    st["u"], st["row"], st["last"] = t_lo, row, st["hi"] == n
                    return True
                if not advance():
                    return False

        if not enter():
            continue
        while True:
            seq, kv, u, hi, row = st["seq"], st["kv"], st["u"], st["hi"], st["row"]
            subs = []
            t = u
            while with_subs and t < hi:
                m = min(MIN_SHARE, hi - t)
                subs.append((t * TILE, min((t + m) * TILE, ln[seq])))
                t += m
            pieces.setdefault((seq, kv), []).append((w, row, u, hi, subs))
            if st["last"] and row + 1 < P:
                marks[(seq, kv)] = row + 1
            if not (advance() and enter()):
                break
    return pieces, marks, ln, tiles_of


def check(lens, hkv, P, G, pair_ratio=200, stream_cost=8, block_size=16, mistake=None, lockstep=False):
    pieces, marks, ln, tiles_of = balanced_schedule(lens, hkv, P, G, pair_ratio, stream_cost, mistake,
                                                    lockstep=lockstep)
    max_rows = 0
    for s in range(len(lens)):
        for kv in range(hkv):
            key = (s, kv)
            if ln[s] == 0:
                assert key not in pieces
                continue
            assert key in pieces, key
            ps = sorted(pieces[key], key=lambda p: p[2])
            if lockstep:  # every KV head of the sequence takes the same pieces (groups, rows, tiles)
                assert [p[:4] for p in ps] == [p[:4] for p in sorted(pieces[(s, 0)], key=lambda p: p[2])], key
            pos = 0
            for _, _, t_lo, t_hi, subs in ps:
                assert t_lo == pos, (key, ps)
                pos = t_hi
                for start, end in subs:
                    assert end > start
                    assert (end - 1) // block_size - start // block_size + 1 <= 64, "sub-unit spans > 64 blocks"
            assert pos == tiles_of[s], key
            rows = sorted(p[1] for p in ps)
            n = len(rows)
            assert rows == list(range(n)), (key, rows)
            assert n <= P, (key, n, P)
            if n < P:
                assert marks.get(key) == n, (key, n, marks.get(key))
            max_rows = max(max_rows, n)
    return max_rows


def llama_lens():
    rng = random.Random(0)
    return [rng.randint(512, 4096) for _ in range(64)]


@pytest.mark.parametrize(
    "name,lens,hkv,P,G,ratio",
    [
        ("c2_llama3_8b_b64", llama_lens(), 8, 8, 512, 200),
        ("c3_128k_b1", [131072], 8, 256, 512, 200),
        ("c3_128k_b4", [131072] * 4, 8, 256, 512, 200),
        ("c5_stress", [0, 1, 32768, 5000, 17, 512, 513] * 36, 2, 64, 512, 100),  # 2-wave workgroups: ratio 1
        ("one_stream_140k", [140000], 1, 274, 512, 200),
        ("one_stream_270k", [270000], 1, 528, 512, 200),
        ("fp8_three_per_cu", llama_lens(), 8, 8, 768, 100),
        ("small_llama_b32_2048", [2048] * 32, 8, 4, 512, 200),
        ("small_llama_b8_8192", [8192] * 8, 8, 16, 512, 200),
        ("small_qwen7b_b64", llama_lens(), 4, 8, 512, 200),
    ],
)
@pytest.mark.parametrize("lockstep", [False, True])
def test_benchmark_shapes(name, lens, hkv, P, G, ratio, lockstep):
    rows = check(lens, hkv, P, G, ratio, stream_cost=12 if name.startswith("fp8") else 8, lockstep=lockstep)
    if name == "c3_128k_b1" and not lockstep:  # lockstep: 64 groups, at most one piece each
        assert rows > 64
    if name == "one_stream_140k":
        assert rows > 64
    if name == "one_stream_270k":
        assert rows > 128


def test_random_shapes():
    rng = random.Random(7)
    for _ in range(400):
        S = rng.choice([1, 2, 3, 5, 17, 64, 300])
        P = rng.choice([2, 3, 4, 5, 8, 9, 64, 256])
        maxl = P * PART
        mode = rng.random()
        lens = []
        for _ in range(S):
            if mode < 0.3:
                x = rng.randint(0, maxl)
            elif mode < 0.6:
                x = rng.choice([0, 1, 15, 16, 17, 511, 512, 513, 1023, 1024, 1025, maxl - 1, maxl, maxl + 100])
            else:
                x = int(math.exp(rng.random() * math.log(maxl + 1)))
            lens.append(x)
        if sum(lens) == 0:
            lens[0] = 1
        hkv = rng.choice([1, 2, 4, 5, 8])
        grid = rng.choice([1, 2, 7, 64, 256, 510, 512, 768, 1024])
        lockstep = grid % hkv == 0 and grid // hkv >= 2 and rng.random() < 0.5  # the host's condition
        check(lens, hkv, P, grid, rng.choice([100, 150, 200, 240]), rng.choice([0, 1, 8, 12, 70]),
              rng.choice([16, 32, 48]), lockstep=lockstep)


@pytest.mark.parametrize("mistake,lockstep", [("row", False), ("end", False), ("row", True), ("end", True),
                                              ("head", True)])
def test_planted_mistake_is_caught(mistake, lockstep):
    """Row numbers anchored on a stream's overhead instead of its first tile
    (a stream whose overhead starts in the previous share gets no row 0), a
    piece that stops one tile short, or lockstep workgroups that all walk the
    group's first KV head, must fail the checks."""
    lens = llama_lens()
    check(lens, 8, 8, 512, lockstep=lockstep)
    with pytest.raises(AssertionError):
        check(lens, 8, 8, 512, mistake=mistake, lockstep=lockstep)


@pytest.mark.parametrize("G", [512, 768])
@pytest.mark.parametrize("lockstep", [False, True])
def test_largest_balanced_launch_keeps_32_bit_boundaries(G, lockstep):
    """The host takes the balanced schedule while sequences x KV heads x
    partitions x 32 tiles < 2^30: at 2048 sequences of the longest length the
    cost line is just below that, and every share boundary still fits."""
    P = (2**30 // (2048 * 8 * 32)) - 1
    lens = [P * PART] * 2048
    assert 2048 * 8 * P * (PART // TILE) < 2**30
    pieces, _, _, tiles_of = balanced_schedule(lens, 8, P, G, 200 if G == 512 else 100, 12, with_subs=False,
                                               lockstep=lockstep)
    assert sum(hi - lo for ps in pieces.values() for _, _, lo, hi, _ in ps) == 8 * sum(tiles_of)


@pytest.mark.parametrize("lens,hkv,P", [([2048] * 32, 8, 4), ([8192] * 8, 8, 16), ([1500] * 40, 8, 3)])
def test_small_totals_keep_both_halves_busy(lens, hkv, P):
    """Cost lines too short for a 2:1 first-half ratio above the minimum share:
    at least as many workgroups of the second half get work as the minimum
    share allows, so the grid is not left half idle. Keeping the ratio with
    the second half raised to the minimum (a planted mistake) fails this."""
    def busy_second_half(mistake=None):
        pieces, _, _, _ = balanced_schedule(lens, hkv, P, 512, 200, 8, mistake=mistake, with_subs=False)
        return len({w for ps in pieces.values() for w, *_ in ps if w >= 256})

    total = sum(((min(x, P * PART) + TILE - 1) // TILE + 8) * hkv for x in lens)
    expect = min(256, max(0, total - 256 * MIN_SHARE) // MIN_SHARE)  # second-half shares the work fills
    assert busy_second_half() >= expect
    assert busy_second_half("clamp") < expect
    check(lens, hkv, P, 512)
