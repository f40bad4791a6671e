"""The C-ABI library on the CPU: it loads, exports every symbol include/varlen_attn.h declares,
plans work correctly and rejects bad arguments before any GPU call."""

import ctypes
import os
import re

import numpy as np
import pytest

from hackaton_amd import _lib
from hackaton_amd.attention import build_plan_host

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "varlen_attn.h")


def doc_tiles(lengths):
    """128-row tiles of the documents (empty ones have none)."""
    return sum(-(-int(x) // 128) for x in lengths if int(x) > 0)


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(va_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert lib.va_abi_version() == 1
    assert lib.va_head_dim() == 128


def plan(lengths, hq, hkv, kind):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return cu, build_plan_host(cu, hq, hkv, kind)


@pytest.mark.parametrize("lengths", [[512] * 4, [64, 37, 50, 12], [1, 1, 1], [129, 0, 300],
                                     [4096, 17]])
@pytest.mark.parametrize("hq,hkv", [(12, 2), (28, 4), (12, 12)])
def test_forward_plan_covers_every_query_tile_once(lengths, hq, hkv):
    cu, items = plan(lengths, hq, hkv, _lib.VA_PLAN_FWD)
    seen = set()
    for q0, doc_end, doc_start, h in items.tolist():
        assert 0 <= h < hq
        d = int(np.searchsorted(cu, doc_start, side="right")) - 1
        assert cu[d] == doc_start and cu[d + 1] == doc_end  # never crosses a document
        assert doc_start <= q0 < doc_end and (q0 - doc_start) % 128 == 0
        seen.add((q0, h))
    expected = {(q0, h) for s, e in zip(cu[:-1], cu[1:]) for q0 in range(s, e, 128)
                for h in range(hq)}
    assert seen == expected and len(items) == len(expected)
    check_xcd_order(items, hq, hkv, lambda q0, e, s, w: min(q0 + 128, e) - s)


NARROW = 1 << 22  # item word bit of a narrow (64-query) forward item


@pytest.mark.parametrize("lengths", [[512] * 4, [64, 37, 50, 12], [1, 1, 1], [129, 0, 300],
                                     [4096, 17], [450, 450, 60], [100, 450]])
@pytest.mark.parametrize("hq,hkv", [(12, 2), (28, 4), (12, 12)])
def test_narrow_forward_plan_splits_the_longest_items_of_short_lists(lengths, hq, hkv):
    """VA_PLAN_FWD_NARROW: when (T + the number of longest documents) x Hq <= 256 (T = the sum of
    ceil(length / 128)), the last 128-query tile of every document of the maximal length becomes
    narrow items of 64 queries (the second only where the tile has more than 64 queries), and
    every (query, head) is still covered once; otherwise the list is VA_PLAN_FWD's."""
    cu, plain = plan(lengths, hq, hkv, _lib.VA_PLAN_FWD)
    _, items = plan(lengths, hq, hkv, _lib.VA_PLAN_FWD_NARROW)
    longest = max(lengths)
    tiles = sum(-(-x // 128) for x in lengths if x > 0)
    split = (tiles + lengths.count(longest)) * hq <= 256
    covered = set()
    for q0, e, s, w in items.tolist():
        h = w & ~NARROW
        assert 0 <= h < hq and w & ~(NARROW | 0xFFF) == 0
        n = 64 if w & NARROW else 128
        if w & NARROW:
            assert split and e - s == longest and e - q0 <= 128 and (q0 - s) % 64 == 0
        else:
            assert (q0 - s) % 128 == 0 and not (split and e - s == longest and q0 + 128 >= e)
        covered.update((q, h) for q in range(q0, min(q0 + n, e)))
    assert len(covered) == sum(lengths) * hq
    assert sum(min(q0 + (64 if w & NARROW else 128), e) - q0 for q0, e, s, w in
               items.tolist()) == sum(lengths) * hq  # no query twice
    if not split:
        assert items.tolist() == plain.tolist()
    else:
        assert len(items) <= 256
        # the planner's work measure of a narrow item is its whole tile's (both halves alike)
        check_xcd_order(items, hq, hkv,
                        lambda q0, e, s, w: (e if w & NARROW else min(q0 + 128, e)) - s)
    cap = ctypes.c_int64()
    assert _lib.lib().va_plan_capacity(sum(lengths), len(lengths), hq, _lib.VA_PLAN_FWD_NARROW,
                                       ctypes.byref(cap)) == _lib.VA_OK
    tiles_cap = -(-sum(lengths) // 128) + len(lengths)
    assert len(items) <= cap.value == max(tiles_cap * hq, min(256, (tiles_cap + len(lengths)) * hq))


def test_configuration_2_forward_list_splits_its_48_longest_items():
    """At configuration 2 (4 x 512 tokens, 12 heads) the 48 items over 512 keys become 96 narrow
    items: 240 items for 256 CUs."""
    _, items = plan([512] * 4, 12, 2, _lib.VA_PLAN_FWD_NARROW)
    narrow = items[(items[:, 3] & NARROW) != 0]
    assert len(items) == 240 and len(narrow) == 96
    assert sorted(set((narrow[:, 0] - narrow[:, 2]).tolist())) == [384, 448]


HEAD_MASK = (1 << 12) - 1  # item word: kind << 24 | group << 21 | pair << 20 | (S-1) << 12 | head


def check_xcd_order(items, hq, hkv, work_of, per_combo=None):
    """The items of one (tile, kind, GQA group, work) sit a constant stride apart, at most 8 (the
    XCD count: work-group i runs on XCD i mod 8, so they share one L2), `per_combo` of them
    (default G = Hq / Hkv: one per head), and the groups come longest first."""
    g = hq // hkv
    combos = {}
    for pos, (a, e, s, w) in enumerate(items.tolist()):
        work = work_of(a, e, s, w)
        key = (a, e, s, w >> 24, (w & HEAD_MASK) // g, work)
        combos.setdefault(key, []).append((pos, work))
    firsts = []
    for key, entries in combos.items():
        expect = g if per_combo is None else per_combo(key)
        assert len(entries) == expect, (key, len(entries), expect)
        pos = [p for p, _ in entries]
        steps = {b - a for a, b in zip(pos, pos[1:])}
        assert len(steps) <= 1 and all(0 < x <= 8 for x in steps), (key, pos)
        firsts.append((pos[0], entries[0][1]))
    work = [w for _, w in sorted(firsts)]
    assert work == sorted(work, reverse=True)


def test_backward_plan_deals_every_xcd_the_same_items():
    """Four 512-token documents: work-group i runs on XCD i mod 8, and every XCD gets the same
    mix of item kinds and spans. (With no per-item cost in the work measure, kv items over 384
    queries tie with q items over 512 keys, and the block layout sent all of the former to half
    of the XCDs.)"""
    hq, hkv = 12, 2
    _, items = plan([512] * 4, hq, hkv, _lib.VA_PLAN_BWD)
    mixes = []
    for x in range(8):
        mix = sorted((w >> 24, (e - a) if w >> 24 == 0 else min(a + 128, e) - s)
                     for a, e, s, w in items[x::8].tolist())
        mixes.append(mix)
    assert all(m == mixes[0] for m in mixes)


def group_heads(w):
    """S of a group item (its heads h .. h + S - 1)."""
    return ((w >> 12) & 0xFF) + 1


def bwd_work(a, e, s, w):
    """The planners' measure: MFMAs per wave per iteration + item cost (a pair item's halves each
    take every step of one head; a per-head item's halves take alternate steps; a group item's
    halves alternate over its S heads' steps)."""
    if w >> 24 == 0:
        steps = (e - a + 31) // 32
        if (w >> 21) & 1:
            return (group_heads(w) * steps + 1) // 2 * 32 + 39
        return (steps if (w >> 20) & 1 else (steps + 1) // 2) * 32 + 39
    return ((min(a + 128, e) - s + 31) // 32 + 1) // 2 * (48 if (w >> 20) & 1 else 24) + 30


@pytest.mark.parametrize("lengths", [[512] * 4, [64, 37, 50, 12], [1], [257, 3]])
@pytest.mark.parametrize("hq,hkv", [(12, 2), (28, 4), (12, 12)])
@pytest.mark.parametrize("kind", [_lib.VA_PLAN_BWD, _lib.VA_PLAN_BWD_HEADS,
                                  _lib.VA_PLAN_BWD_PAIRS])
def test_backward_plan_covers_every_key_and_query_tile_once(lengths, hq, hkv, kind):
    """kv items (dK/dV of 128 keys) and q items (dQ of 128 queries) cover every (tile, head) once:
    one head each (heads plans) or two heads of one GQA group, the last head of an odd group
    alone (pairs plans)."""
    g = hq // hkv
    bound = 2 * doc_tiles(lengths) * hq
    pairs = g > 1 and (kind == _lib.VA_PLAN_BWD_PAIRS or
                       (kind == _lib.VA_PLAN_BWD and bound >= _lib.VA_BWD_PAIR_MIN_ITEMS))
    cu, items = plan(lengths, hq, hkv, kind)
    kv_seen, q_seen = [], []
    for a, doc_end, doc_start, w in items.tolist():
        item_kind, pair, h = w >> 24, (w >> 20) & 15, w & HEAD_MASK
        assert 0 <= h < hq and item_kind in (0, 1) and pair in (0, 1)
        d = int(np.searchsorted(cu, doc_start, side="right")) - 1
        assert cu[d] == doc_start and cu[d + 1] == doc_end
        assert doc_start <= a < doc_end and (a - doc_start) % 128 == 0
        seen = kv_seen if item_kind == 0 else q_seen
        if pair:
            assert pairs and (h % g) % 2 == 0 and (h % g) + 1 < g
            seen += [(a, h), (a, h + 1)]
        else:
            assert not pairs or h % g == g - 1, "pair plans keep only an odd group's last head"
            seen.append((a, h))
    expected = sorted((t, h) for s, e in zip(cu[:-1], cu[1:]) for t in range(s, e, 128)
                      for h in range(hq))
    assert sorted(kv_seen) == expected and sorted(q_seen) == expected
    n_kind = len(expected) // hq * hkv * ((g + 1) // 2 if pairs else g)
    assert len(items) == 2 * n_kind
    if pairs:
        def per_combo(key):  # a group's pair items, the odd group's single, or both at one work
            a, e, s, item_kind, _grp, work = key
            single = bwd_work(a, e, s, item_kind << 24)
            pair = bwd_work(a, e, s, (item_kind << 24) | (1 << 20))
            if g % 2 == 0:
                return g // 2
            if pair == single:
                return (g + 1) // 2
            return 1 if work == single else g // 2
        check_xcd_order(items, hq, hkv, bwd_work, per_combo)
    else:
        check_xcd_order(items, hq, hkv, bwd_work)


@pytest.mark.parametrize("lengths", [[512] * 4, [64, 37, 50, 12], [1], [257, 3], [1000, 24, 300],
                                     [180] * 45, [1740, 400, 90]])
@pytest.mark.parametrize("hq,hkv", [(12, 2), (28, 4), (12, 12), (4, 1)])
@pytest.mark.parametrize("kind", [_lib.VA_PLAN_BWD_GROUPS, _lib.VA_PLAN_BWD_GROUPS_ALL])
def test_group_plan_covers_every_tile_once(lengths, hq, hkv, kind):
    """Group plans: the kv items cover every (key tile, query head) exactly once, a key tile either
    by group items (bit 21) of S heads each, S >= 2 dividing G, G / S per GQA group, or by the
    VA_PLAN_BWD items of that tile; the q items are VA_PLAN_BWD's. VA_PLAN_BWD_GROUPS gives a
    tile the largest S whose group item does no more work than the VA_PLAN_BWD list's longest
    item or its work per CU (256), and no group item when none does, S < G only in lists long
    enough to take pair items; VA_PLAN_BWD_GROUPS_ALL gives every tile S = G; with Hq == Hkv both
    are VA_PLAN_BWD."""
    g = hq // hkv
    cu, items = plan(lengths, hq, hkv, kind)
    _, base = plan(lengths, hq, hkv, _lib.VA_PLAN_BWD)
    if g == 1:
        assert np.array_equal(items, base)
        return
    base_works = [bwd_work(*x) for x in base.tolist()]
    cap = max(max(base_works), sum(base_works) // 256)
    covered, subsets = [], {}
    for a, e, s, w in items.tolist():
        if w >> 24 != 0:
            continue
        h = w & HEAD_MASK
        if (w >> 21) & 1:
            n = group_heads(w)
            assert n >= 2 and g % n == 0 and h % n == 0 and not (w >> 20) & 1
            subsets.setdefault((a, e, s), set()).add(n)
            covered += [(a, x) for x in range(h, h + n)]
        elif (w >> 20) & 1:
            covered += [(a, h), (a, h + 1)]
        else:
            covered.append((a, h))
    expected = sorted((t, h) for s0, e0 in zip(cu[:-1], cu[1:]) for t in range(s0, e0, 128)
                      for h in range(hq))
    assert sorted(covered) == expected
    for (a, e, s), ns in subsets.items():
        assert len(ns) == 1, (a, ns)  # one head count per tile
    bound = 2 * doc_tiles(lengths) * hq
    pairs = bound >= _lib.VA_BWD_PAIR_MIN_ITEMS
    for a, e, s in {(a, e, s) for a, e, s, w in items.tolist() if w >> 24 == 0}:
        steps = (e - a + 31) // 32
        fits = [n for n in range(g, 1, -1) if g % n == 0 and (n * steps + 1) // 2 * 32 + 39 <= cap
                and (pairs or n == g)]
        want = g if kind == _lib.VA_PLAN_BWD_GROUPS_ALL else (fits[0] if fits else None)
        assert subsets.get((a, e, s), {None}) == {want}, (a, e, s, want)
    plain = [tuple(x) for x in base.tolist() if x[3] >> 24 == 1 or tuple(x[:3]) not in subsets]
    assert sorted(plain) == sorted(tuple(x) for x in items.tolist() if not (x[3] >> 21) & 1)

    def per_combo(key):  # G / S group items; otherwise as in the VA_PLAN_BWD list
        a, e, s, item_kind, _grp, work = key
        if item_kind == 0 and (a, e, s) in subsets:
            return g // next(iter(subsets[(a, e, s)]))
        if not pairs:
            return g
        single = bwd_work(a, e, s, item_kind << 24)
        pair = bwd_work(a, e, s, (item_kind << 24) | (1 << 20))
        if g % 2 == 0:
            return g // 2
        if pair == single:
            return (g + 1) // 2
        return 1 if work == single else g // 2
    check_xcd_order(items, hq, hkv, bwd_work, per_combo)


@pytest.mark.parametrize("lengths,pairs", [([512] * 4, False), ([64, 37, 50, 12], False),
                                           ([4096, 4096], True), ([180] * 45, True),
                                           ([100] * 42, False), ([100] * 43, True),
                                           ([0] * 50 + [100] * 42, False)])
def test_backward_plan_takes_pairs_when_the_list_is_long(lengths, pairs):
    """VA_PLAN_BWD is the heads plan below VA_BWD_PAIR_MIN_ITEMS per-head items (2 T Hq, T the
    128-row tiles of the documents, a count the device planner makes from the same bounds) and
    the pairs plan from there on."""
    hq, hkv = 12, 2
    bound = 2 * doc_tiles(lengths) * hq
    assert (bound >= _lib.VA_BWD_PAIR_MIN_ITEMS) == pairs
    _, auto = plan(lengths, hq, hkv, _lib.VA_PLAN_BWD)
    _, fixed = plan(lengths, hq, hkv, _lib.VA_PLAN_BWD_PAIRS if pairs else _lib.VA_PLAN_BWD_HEADS)
    assert np.array_equal(auto, fixed)


def test_plan_rejects_bad_cu_seqlens():
    lib = _lib.lib()
    n = ctypes.c_int64()
    for cu, code in (([1, 5], _lib.VA_ESEQ), ([0, 5, 3], _lib.VA_ESEQ)):
        arr = np.asarray(cu, dtype=np.int32)
        rc = lib.va_plan_size(arr.ctypes.data_as(_lib._pi32), len(cu) - 1, 12, 2, 0,
                              ctypes.byref(n))
        assert rc == code
        assert b"cu_seqlens" in lib.va_last_error()
    arr = np.asarray([0, 5], dtype=np.int32)
    assert lib.va_plan_size(arr.ctypes.data_as(_lib._pi32), 1, 12, 5, 0,
                            ctypes.byref(n)) == _lib.VA_ESHAPE
    assert lib.va_plan_size(arr.ctypes.data_as(_lib._pi32), 1, 12, 2, 7,
                            ctypes.byref(n)) == _lib.VA_EINVAL
    small = np.zeros((1, 4), dtype=np.int32)
    rc = lib.va_plan_build(arr.ctypes.data_as(_lib._pi32), 1, 12, 2, 0,
                           small.ctypes.data_as(_lib._pi32), 1, ctypes.byref(n))
    assert rc == _lib.VA_ECAPACITY and n.value == 12


def test_attention_entry_points_validate_before_launching():
    """Argument errors come back as codes with a message; no GPU is touched."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc = lib.va_fwd(fake, fake, fake, fake, fake, fake, 4, 100, 12, 2, 64, 0.1, 0, None)
    assert rc == _lib.VA_ESHAPE and b"head_dim" in lib.va_last_error()
    rc = lib.va_fwd(fake, fake, fake, fake, fake, fake, 4, 100, 12, 5, 128, 0.1, 0, None)
    assert rc == _lib.VA_ESHAPE
    rc = lib.va_fwd(fake, fake, fake, fake, fake, fake, 4, 100, 12, 2, 128, 0.1, 9, None)
    assert rc == _lib.VA_EDTYPE
    rc = lib.va_fwd(fake, None, fake, fake, fake, fake, 4, 100, 12, 2, 128, 0.1, 0, None)
    assert rc == _lib.VA_EINVAL
    rc = lib.va_fwd(fake, ctypes.c_void_p(0x1008), fake, fake, fake, fake, 4, 100, 12, 2, 128,
                    0.1, 0, None)
    assert rc == _lib.VA_EINVAL and b"aligned" in lib.va_last_error()
    rc = lib.va_fwd(fake, fake, fake, fake, fake, fake, 4, 100, 12, 2, 128, float("nan"), 0,
                    None)
    assert rc == _lib.VA_EINVAL
    rc = lib.va_fwd(fake, fake, fake, fake, fake, fake, 4, 100, 12, 2, 128, -0.5, 0, None)
    assert rc == _lib.VA_EINVAL and b"positive" in lib.va_last_error()
    # nothing to do is not an error
    assert lib.va_fwd(None, None, None, None, None, None, 0, 0, 12, 2, 128, 0.1, 0, None) == 0
    offs = (ctypes.c_int64 * 2)()
    nbytes = ctypes.c_int64()
    assert lib.va_bwd_workspace_layout(2048, 12, 2, 128, offs, ctypes.byref(nbytes)) == 0
    assert list(offs) == [0, 2048 * 12 * 256]
    # partials, then one flag per row, then the row statistics (two fp32 per query head and row)
    assert nbytes.value == 2 * 2048 * 12 * 256 + 2048 * 4 + 2048 * 12 * 8
    rc = lib.va_bwd(fake, fake, fake, fake, fake, fake, fake, 4, 2048, 12, 2, 128, 0.1, 0, fake,
                    None, None, fake, nbytes.value - 1, None)
    assert rc == _lib.VA_ECAPACITY
    rc = lib.va_bwd(fake, fake, fake, fake, fake, fake, fake, 4, 2048, 12, 2, 128, 0.1, 0, fake,
                    fake, None, fake, nbytes.value, None)
    assert rc == _lib.VA_EINVAL and b"both" in lib.va_last_error()
    for stage in (0, 6):  # stages 1-5 exist
        rc = lib.va_bwd_stage(stage, fake, fake, fake, fake, fake, fake, fake, 4, 2048, 12, 2, 128,
                              0.1, 0, fake, fake, fake, fake, nbytes.value, None)
        assert rc == _lib.VA_EINVAL and b"stage" in lib.va_last_error()
    rc = lib.va_rope_fwd(fake, fake, fake, fake, fake, 0, 128, fake, fake, fake, fake, fake, 10,
                         12, 2, 128, 0, 0, 0, 1, 0, None)
    assert rc == _lib.VA_EINVAL  # padded layout needs seq > 0
    rc = lib.va_pack_rows(fake, fake, fake, fake, 10, 12, 64, 127, 2, 0, None)
    assert rc == _lib.VA_ESHAPE


def test_product_path_refuses_cpu_tensors():
    import torch

    from hackaton_amd import varlen_attention
    q = torch.zeros(8, 12, 128, dtype=torch.float16)
    k = torch.zeros(8, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU only"):
        varlen_attention(q, k, k, [8], 0.1)


@pytest.mark.parametrize("lengths", [[512] * 4, [64, 37, 50, 12], [1, 1, 1], [129, 0, 300],
                                     [4096, 17], [127, 128, 129]])
@pytest.mark.parametrize("kind", [_lib.VA_PLAN_FWD, _lib.VA_PLAN_BWD, _lib.VA_PLAN_BWD_HEADS,
                                  _lib.VA_PLAN_BWD_PAIRS, _lib.VA_PLAN_BWD_GROUPS,
                                  _lib.VA_PLAN_BWD_GROUPS_ALL])
def test_device_plan_capacity_bounds_the_host_plan(lengths, kind):
    """va_plan_capacity, from host-known sizes only, is never below the real item count."""
    hq = 12
    cu, items = plan(lengths, hq, 2, kind)
    cap = np.zeros(1, dtype=np.int64)
    assert _lib.lib().va_plan_capacity(int(cu[-1]), len(lengths), hq, kind,
                                       cap.ctypes.data_as(_lib._pi64)) == 0
    assert int(cap[0]) >= len(items)
    tiles = -(-int(cu[-1]) // 128) + len(lengths)
    assert int(cap[0]) == tiles * hq * (1 if kind == _lib.VA_PLAN_FWD else 2)


def test_device_plan_rejects_bad_arguments_before_launching():
    lib = _lib.lib()
    cap = np.zeros(1, dtype=np.int64)
    p = cap.ctypes.data_as(_lib._pi64)
    assert lib.va_plan_capacity(100, 9000, 12, _lib.VA_PLAN_FWD, p) == _lib.VA_ESHAPE  # > 8192
    assert lib.va_plan_capacity(-1, 1, 12, _lib.VA_PLAN_FWD, p) == _lib.VA_ESHAPE
    assert lib.va_plan_capacity(100, 1, 12, 7, p) == _lib.VA_EINVAL
    # capacity below the bound, NULL pointers and bad heads fail before any device call
    assert lib.va_plan_build_device(None, 1, 100, 12, 2, _lib.VA_PLAN_FWD, None, 100,
                                    None) == _lib.VA_EINVAL
    fake = ctypes.c_void_p(4096)
    assert lib.va_plan_build_device(fake, 1, 100, 12, 2, _lib.VA_PLAN_FWD, fake, 1,
                                    None) == _lib.VA_ECAPACITY
    assert lib.va_plan_build_device(fake, 1, 100, 12, 5, _lib.VA_PLAN_FWD, fake, 1000,
                                    None) == _lib.VA_ESHAPE


def test_header_constants_match_python():
    """Every enum constant of include/varlen_attn.h has the same value in hackaton_amd._lib."""
    import re
    from pathlib import Path

    text = (Path(__file__).resolve().parent.parent / "include" / "varlen_attn.h").read_text()
    consts = {}
    for body in re.findall(r"enum\s*\{([^}]*)\}", text):
        for name, value in re.findall(r"(VA_\w+)\s*=\s*(-?\d+)", body):
            consts[name] = int(value)
    assert "VA_FWD_MANY_ITEMS" in consts and "VA_PLAN_BWD" in consts
    for name, value in consts.items():
        if hasattr(_lib, name):
            assert getattr(_lib, name) == value, name


def test_backward_workspace_only_where_partials_exist():
    """Hq == Hkv with dK/dV returned (the reference's expanded call) needs no workspace: the
    kernels write dK/dV directly, so the Python layer allocates none (448 MiB of unused partials
    at N = 32768, H = 28 otherwise)."""
    from hackaton_amd.attention import bwd_workspace_needed

    assert not bwd_workspace_needed(12, 12)
    assert not bwd_workspace_needed(28, 28, outputs=True)
    assert bwd_workspace_needed(12, 12, outputs=False)  # the partials are the result
    assert bwd_workspace_needed(12, 2)
    assert bwd_workspace_needed(28, 4, outputs=False)


def test_noalloc_refuses_sizes_beyond_its_scratch():
    """va_bwd_noalloc checks sizes and arguments on the host before any launch or device query;
    the fake pointers are never dereferenced."""
    lib = _lib.lib()
    scale = 128 ** -0.5
    limit = lib.va_bwd_noalloc_max_bytes() // (2 * 2 * 128)  # tokens x query heads it holds
    fake = ctypes.c_void_p(0x1000)
    n = limit // 12 + 1
    rc = lib.va_bwd_noalloc(fake, fake, fake, fake, fake, fake, fake, 4, n, 12, 2, 128, scale, 0,
                            fake, fake, fake, None)
    assert rc == _lib.VA_ECAPACITY
    assert b"scratch" in lib.va_last_error()
    rc = lib.va_bwd_noalloc(fake, fake, fake, fake, fake, fake, fake, 4, 100, 12, 2, 128, scale, 0,
                            fake, None, None, None)
    assert rc == _lib.VA_EINVAL
    assert limit >= 8192 * 12  # configurations 2 and 3 fit


def test_ceiling_probes_check_arguments_before_any_launch():
    """va_probe_mfma / va_probe_copy refuse bad arguments on the host (the fake pointers are never
    dereferenced, nothing is launched)."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    assert lib.va_probe_mfma(_lib.VA_F32, 1, 1, fake, None) == _lib.VA_EDTYPE
    assert lib.va_probe_mfma(_lib.VA_F16, 0, 1, fake, None) == _lib.VA_EINVAL
    assert lib.va_probe_mfma(_lib.VA_F16, 1, 0, fake, None) == _lib.VA_EINVAL
    assert lib.va_probe_mfma(_lib.VA_BF16, 1, 1, None, None) == _lib.VA_EINVAL
    assert lib.va_probe_copy(None, fake, 16, 1, None) == _lib.VA_EINVAL
    assert lib.va_probe_copy(fake, fake, 24, 1, None) == _lib.VA_EINVAL
    assert lib.va_probe_copy(fake, fake, 16, 0, None) == _lib.VA_EINVAL
    assert lib.va_probe_copy(ctypes.c_void_p(0x1008), fake, 16, 1, None) == _lib.VA_EINVAL
    assert lib.va_probe_copy(fake, fake, 0, 1, None) == _lib.VA_OK  # nothing to copy


def test_row_statistics_rule():
    """va_plan_bwd_row_stats: the mean over query rows of the 128-key tiles at or before the
    row's own, against VA_BWD_STATS_MIN_TILES = 3. Closed forms: a document of 128 m rows covers
    its rows (m + 1) / 2 times on average; configurations 1-4 stay below 3, configuration 5's
    long documents (3.44) pass."""
    from hackaton_amd import workloads as wl
    from hackaton_amd.attention import bwd_row_stats

    assert _lib.VA_BWD_STATS_MIN_TILES == 3
    assert not bwd_row_stats([0, 128 * 4])       # mean 2.5
    assert bwd_row_stats([0, 128 * 5])           # mean 3.0
    assert not bwd_row_stats([0, 128 * 5 - 1])   # 127 rows of the last tile short
    assert not bwd_row_stats([0, 128 * 5, 128 * 5 + 1])  # one row more, covered once
    assert not bwd_row_stats([0])                # no documents
    for cfg, expect in ((1, False), (2, False), (3, False), (4, False), (5, True)):
        lengths = wl.config_lengths(cfg)
        assert bwd_row_stats(np.concatenate([[0], np.cumsum(lengths)])) is expect, cfg
    use = ctypes.c_int32(7)
    assert _lib.lib().va_plan_bwd_row_stats(None, 1, ctypes.byref(use)) == _lib.VA_EINVAL


def test_rope_forward_may_leave_the_value_rows_out_only_without_expand():
    """va_rope_fwd takes v = v_out = NULL (value rows left out: the caller uses its v as it is)
    only when nothing is expanded; the backward always needs dv. Checked before any launch."""
    lib = _lib.lib()
    f = ctypes.c_void_p(0x1000)

    def call(fn, v, v_out, expand):
        # (x0, x1, x2, cos, sin, strides, b_idx, t_idx, y0, y1, y2, n, heads, kv_heads, D, seq,
        #  in_dtype, out_dtype, layout, expand, stream)
        return fn(f, f, v, f, f, 0, 128, f, f, f, f, v_out, 10, 12, 2, 128, 0, 0, 0, 0, expand,
                  None)
    rc = call(lib.va_rope_fwd, None, None, 1)
    assert rc == _lib.VA_EINVAL and b"left out" in lib.va_last_error()  # expand = 1
    assert call(lib.va_rope_fwd, f, None, 0) == _lib.VA_EINVAL  # only one of the two
    rc = call(lib.va_rope_bwd, None, None, 0)
    assert rc == _lib.VA_EINVAL and b"left out" in lib.va_last_error()
