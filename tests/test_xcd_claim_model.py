"""A CPU model of xcd_slot (csrc/paged_decode.hip): the claim that gives each workgroup of the
paired balanced kernel an XCD-stable index.

Workgroup w of the aligned block k = w / 8 claims bit x = its XCC_ID of the block's mask word
with an atomic or, or, when that bit is taken, the first free bit; the claim that fills the
mask clears it.  The device code relies on:
  * the 8 workgroups of a block get 8 distinct indices 8k .. 8k+7, whatever XCC_IDs the
    dispatcher gave them and however their atomics interleave (a bijection on every block);
  * a dispatch that deals one workgroup of the block to each XCD gives workgroup w index
    8k + (its XCD), so share 8k + x always runs on XCD x;
  * the mask word is zero again when the launch ends;
  * workgroups of a last, partial block keep their own index;
  * a mask that is not zero at launch (a workspace not zero-filled) makes a claim fail: -1.
A planted mistake (a claim that keeps its XCC bit without checking it) is caught.
"""

from __future__ import annotations

import random

import pytest


def _claims(xccs, masks, k, rng, check_taken=True):
    """The 8 claims of block k as generators: each yields before every atomic and returns its
    slot (or -1)."""
    def claim(xcc):
        slot = xcc & 7
        bit = 1 << slot
        yield
        old = masks[k]
        masks[k] |= bit
        if check_taken and (old & bit):
            for slot in range(8):
                bit = 1 << slot
                if old & bit:
                    continue
                yield
                old = masks[k]
                masks[k] |= bit
                if not (old & bit):
                    break
            else:
                return -1
        if (old | bit) == 0xFF:
            yield
            masks[k] = 0
        return 8 * k + slot
    return [claim(x) for x in xccs]


def launch(n, xcc_of, seed=0, masks=None, check_taken=True):
    """Indices of n workgroups; xcc_of(w) is workgroup w's XCC_ID."""
    rng = random.Random(seed)
    nblocks = n // 8
    masks = masks if masks is not None else [0] * nblocks
    result = {}
    gens = {}
    for k in range(nblocks):
        for j, g in enumerate(_claims([xcc_of(8 * k + j) for j in range(8)], masks, k, rng,
                                      check_taken)):
            gens[8 * k + j] = g
    for w in range(nblocks * 8, n):
        result[w] = w                                   # a partial block keeps its own index
    while gens:
        w = rng.choice(list(gens))
        try:
            next(gens[w])
        except StopIteration as stop:
            result[w] = stop.value
            del gens[w]
    return result, masks


@pytest.mark.parametrize("n", [8, 256, 261, 512, 1016])
@pytest.mark.parametrize("start", range(8))
def test_rotated_dispatch_puts_share_8k_plus_x_on_xcd_x(n, start):
    xcc = lambda w: (w + start) % 8
    res, masks = launch(n, xcc, seed=n + start)
    assert sorted(res.values()) == list(range(n))
    for w, idx in res.items():
        if w < n // 8 * 8:
            assert idx % 8 == xcc(w) and idx // 8 == w // 8
    assert all(m == 0 for m in masks)


@pytest.mark.parametrize("seed", range(40))
def test_any_dispatch_gives_a_bijection_and_clears_the_masks(seed):
    r = random.Random(seed)
    n = r.choice([8, 64, 256, 300, 512])
    kind = r.choice(["random", "one_xcd", "pairs"])
    table = {"random": [r.randrange(8) for _ in range(n)],
             "one_xcd": [3] * n,                         # e.g. a partition with one XCD
             "pairs": [(w // 2) % 8 for w in range(n)]}[kind]
    res, masks = launch(n, lambda w: table[w], seed=seed)
    assert sorted(res.values()) == list(range(n)), kind
    assert all(m == 0 for m in masks), kind


def test_a_mask_left_set_makes_claims_fail():
    masks = [0xFF, 0]
    res, masks = launch(16, lambda w: w % 8, masks=masks)
    assert [res[w] for w in range(8)] == [-1] * 8
    assert sorted(res[w] for w in range(8, 16)) == list(range(8, 16))
    assert masks == [0xFF, 0]


def test_planted_mistake_claim_without_checking_is_caught():
    """Keeping the XCC bit without looking at the old mask duplicates indices when two
    workgroups of a block report the same XCD."""
    res, _ = launch(8, lambda w: 5 if w < 2 else w, check_taken=False)
    assert sorted(res.values()) != list(range(8))
