"""A CPU model of the balanced kernel's schedule and of both kernels' merge trees.

The control logic of `mx_paged_decode_balanced` (csrc/paged_decode.hip: the balanced line, the
share of each workgroup, the unit walk, the piece and slot numbering) and of `merge_tree` (the
fan-in-8 arrival counters) is restated here in integer Python, and run over random batches
with the workgroups interleaved at random between pieces and between arrivals.  The checks are
the invariants the device code relies on:
  * every chunk of every unit is streamed exactly once;
  * the workgroups that hold pieces of a unit agree on the unit's first workgroup and piece
    count, and its pieces are items 0 .. n-1, each held once;
  * slots stay below groups + units and are disjoint between units;
  * a merge never reads an item that has not been written, each unit gets exactly one final
    write, and every counter is back at zero when the launch ends;
  * a unit cut in two is merged by its first piece's workgroup without storing that piece
    (merge_first_of_two) only once the second piece has been written and counted, and
    otherwise through the tree as before.
Line constants as in the kernel: 8 positions per chunk (16 for a pair of KV heads) and 64 per
unit; the uniform-batch rule; shares of at least one chunk's weight.
"""

from __future__ import annotations

import math
import random

import pytest

CHUNK = 16
FAN = 8
LEVELS = 4


def _tree(counters, written, finals, unit, slot0, item, nitems, rng_yield):
    """merge_tree for one arrival: yields at each arrival point; returns when this arrival is
    not the last of its group, or after the final write."""
    stride = 1
    for level in range(LEVELS):
        grp = item // FAN
        gsize = min(FAN, nitems - grp * FAN)
        gslot = slot0 + grp * FAN * stride
        yield
        prev = counters[level].get(gslot, 0)
        counters[level][gslot] = prev + 1
        if prev != gsize - 1:
            return
        counters[level][gslot] = 0
        for t in range(gsize):
            assert written.get((level, gslot + t * stride)), \
                f"merge of unit {unit} reads unwritten level-{level} slot {gslot + t * stride}"
        nnext = (nitems + FAN - 1) // FAN
        if nnext == 1:
            assert unit not in finals
            finals[unit] = "merged"
            return
        written[(level + 1, gslot)] = True
        item, nitems, stride = grp, nnext, stride * FAN
    raise AssertionError("merge tree deeper than its levels")


def balanced_launch(lens, ups, groups, chunk_weight=8, unit_overhead=64, seed=0,
                    first_of_two="checked"):
    """Runs one launch of the balanced schedule's control logic; returns (chunks covered per
    unit, final writes per unit, slots used).  first_of_two: "checked" (the kernel), "off" (no
    direct merge of units cut in two) or "unchecked" (a planted mistake: the first piece merges
    without reading the counter)."""
    B = len(lens)
    rng = random.Random(seed)
    n = [(x + CHUNK - 1) // CHUNK if x > 0 else 0 for x in lens]
    units = B * ups
    wc, alpha = chunk_weight, unit_overhead
    # Uniform batches with k workgroups per unit: each chunk one position, the smallest
    # overhead k divides into the span.
    if groups > units and groups % units == 0:
        lo, hi = min(n), max(n)
        if lo == hi and lo > 0:
            k = groups // units
            wc, alpha = 1, (k - lo % k) % k
    weight = [ups * (nb * wc + alpha) if nb > 0 else 0 for nb in n]
    total = sum(weight)
    covered, finals, slots_of = {}, {}, {}
    counters = [dict() for _ in range(LEVELS)]
    written = {}
    if total == 0:
        return covered, finals, slots_of
    qsz = max((total + groups - 1) // groups, wc)

    def wg_proc(wg):
        x_begin = wg * qsz
        if x_begin >= total:
            return
        x_end = min(x_begin + qsz, total)
        start = 0
        b = -1
        for bb in range(B):
            if weight[bb] > 0 and start <= x_begin < start + weight[bb]:
                b, seq_start = bb, start
                break
            start += weight[bb]
        assert b >= 0
        span = n[b] * wc + alpha
        j = (x_begin - seq_start) // span
        u0 = seq_start + j * span
        while True:
            cpos = u0 + alpha
            ca = min(n[b], -(-max(0, x_begin - cpos) // wc))
            cb = min(n[b], -(-max(0, x_end - cpos) // wc))
            if ca < cb:
                unit = b * ups + j
                last = cpos + (n[b] - 1) * wc
                first_wg = wg if cpos >= x_begin else cpos // qsz
                npieces = (wg if last < x_end else last // qsz) - first_wg + 1
                covered.setdefault(unit, []).append((ca, cb, wg, first_wg, npieces))
                yield  # the piece streams
                if npieces == 1:
                    assert unit not in finals
                    finals[unit] = "direct"
                else:
                    slot0 = first_wg + unit
                    item = wg - first_wg
                    assert 0 <= item < npieces
                    assert slot0 + item < groups + units
                    slots_of.setdefault(unit, set()).add(slot0 + item)
                    direct = False
                    if npieces == 2 and item == 0 and first_of_two != "off":
                        yield  # thread 0 reads the unit's level-0 counter
                        if first_of_two == "unchecked" or counters[0].get(slot0, 0) == 1:
                            assert written.get((0, slot0 + 1)), \
                                f"direct merge of unit {unit} reads an unwritten second piece"
                            counters[0][slot0] = 0
                            assert unit not in finals
                            finals[unit] = "first of two"
                            direct = True
                    if not direct:
                        written[(0, slot0 + item)] = True
                        yield from _tree(counters, written, finals, unit, slot0, item, npieces,
                                         rng)
            u0 += span
            if u0 >= x_end:
                break
            j += 1
            if j == ups:
                j = 0
                b += 1
                while b < B and n[b] == 0:
                    b += 1
                assert b < B, "positions only exist for non-empty sequences"
                span = n[b] * wc + alpha

    gens = {w: wg_proc(w) for w in range(groups)}
    while gens:
        w = rng.choice(list(gens))
        try:
            next(gens[w])
        except StopIteration:
            del gens[w]
    assert all(v == 0 for c in counters for v in c.values()), "counters left non-zero"
    return covered, finals, slots_of


def _check_balanced(lens, ups, groups, chunk_weight=8, seed=0):
    covered, finals, slots_of = balanced_launch(lens, ups, groups, chunk_weight, seed=seed)
    _check_units(lens, ups, covered, finals, slots_of)
    return finals


def _check_units(lens, ups, covered, finals, slots_of):
    n = [(x + CHUNK - 1) // CHUNK if x > 0 else 0 for x in lens]
    for b, nb in enumerate(n):
        for j in range(ups):
            unit = b * ups + j
            if nb == 0:
                assert unit not in covered
                continue
            pieces = sorted(covered[unit])
            # the chunks [0, nb) exactly once, in piece order
            assert pieces[0][0] == 0 and pieces[-1][1] == nb
            assert all(p[1] == q[0] for p, q in zip(pieces, pieces[1:]))
            first = {p[3] for p in pieces}
            counts = {p[4] for p in pieces}
            assert len(first) == 1 and counts == {len(pieces)}, (unit, pieces)
            items = sorted(p[2] - p[3] for p in pieces)
            assert items == list(range(len(pieces)))
            expect = {1: {"direct"}, 2: {"merged", "first of two"}}.get(len(pieces), {"merged"})
            assert finals[unit] in expect, (unit, len(pieces), finals[unit])
    all_slots = [s for v in slots_of.values() for s in v]
    assert len(all_slots) == len(set(all_slots)), "slots shared between units"


@pytest.mark.parametrize("seed", range(60))
def test_balanced_schedule_on_random_batches(seed):
    r = random.Random(seed)
    B = r.choice([1, 2, 5, 17, 64, 130])
    ups = r.choice([1, 2, 4, 7, 8])
    groups = r.choice([1, 3, 7, 64, 256, 512])
    cap = r.choice([40, 700, 8192])
    lens = [r.choice([0, 1, 15, 16, 17, cap, int(math.exp(r.uniform(0, math.log(cap))))])
            for _ in range(B)]
    _check_balanced(lens, ups, groups, chunk_weight=r.choice([8, 16]), seed=seed)


@pytest.mark.parametrize("B,ups,groups,L", [
    (64, 4, 256, 4096),     # config 2 over pairs of KV heads: one unit per workgroup
    (64, 8, 256, 4096),     # single heads: two units per workgroup
    (32, 4, 256, 16384),    # sweep B=32 over pairs: two equal pieces per unit
    (8, 4, 256, 4080),      # uniform, k = 8 pieces per unit
    (3, 1, 4095, 8192),     # the deepest tree the counter region allows
    (1, 4, 256, 32768),     # one sequence cut 64 ways
])
def test_balanced_schedule_on_uniform_batches(B, ups, groups, L):
    _check_balanced([L] * B, ups, groups, chunk_weight=16 if ups == 4 else 8)


def test_ragged_config_shape():
    """Config 4's recipe: 256 sequences, log-uniform lengths with 10 % of 1-15 tokens, 4 KV
    heads, 256 workgroups."""
    r = random.Random(4)
    lens = [r.randint(1, 15) if r.random() < 0.1 else int(math.exp(r.uniform(0, math.log(8192))))
            for _ in range(256)]
    finals = _check_balanced(lens, 4, 256)
    # Units cut in two are common here, and the interleaving lets some be merged directly.
    assert list(finals.values()).count("first of two") > 0


def test_first_of_two_without_the_counter_read_is_caught():
    """A planted mistake: the first piece of a unit cut in two merging without reading the
    counter reads an unwritten second piece under some interleaving (or, when the second piece
    was written but not yet counted, leaves its counter non-zero)."""
    r = random.Random(4)
    lens = [r.randint(1, 15) if r.random() < 0.1 else int(math.exp(r.uniform(0, math.log(8192))))
            for _ in range(256)]
    caught = 0
    for seed in range(20):
        try:
            balanced_launch(lens, 4, 256, seed=seed, first_of_two="unchecked")
        except AssertionError as e:
            assert "unwritten second piece" in str(e) or "counters left non-zero" in str(e)
            caught += 1
    assert caught > 0
    # and the checked form agrees with the plain tree on every interleaving tried
    for seed in range(20):
        _, finals_off, _ = balanced_launch(lens, 4, 256, seed=seed, first_of_two="off")
        _, finals_on, _ = balanced_launch(lens, 4, 256, seed=seed)
        assert set(finals_off) == set(finals_on)


@pytest.mark.parametrize("splits", [2, 7, 8, 9, 64, 65, 511, 4096])
def test_split_tree_merges_every_split_once(splits):
    """The split grid's tree: level-0 item s is split s of one unit; arrivals in random order."""
    for seed in range(5):
        rng = random.Random(seed)
        counters = [dict() for _ in range(LEVELS)]
        written, finals = {}, {}
        gens = {}
        for s in range(splits):
            written[(0, s)] = True
            gens[s] = _tree(counters, written, finals, 0, 0, s, splits, rng)
        while gens:
            s = rng.choice(list(gens))
            try:
                next(gens[s])
            except StopIteration:
                del gens[s]
        assert finals == {0: "merged"}
        assert all(v == 0 for c in counters for v in c.values())
