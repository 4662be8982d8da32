"""Pins of the oracle's proximity-factor selection (oracle.c,
orc_proximity_select; cuda_slam/main.cu:1679-1779) by hand-worked cases on a
6-keyframe window (t0 = t1 = 0, rad = 1, nms = 1, thresh = 16) whose edge
lists were derived by hand from the reference's steps: invalidation of
pairs with j > i - rad and of distances above 100, NMS of L1 radius
max(min(|i - j| - 2, nms), 0) around existing and chosen edges, mandatory
neighbour edges (both directions, skipped when (i, j) exists), greedy picks
in ascending distance, the max_factors cut and the final de-duplication.
"""
import numpy as np
import pytest

from oracle import oracle as orc


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


def _d():
    # raw distances; only pairs with j <= i - 3 survive invalidation and seeding
    d = np.full((6, 6), 50.0, np.float32)
    d[3, 0], d[4, 0], d[4, 1] = 5.0, 20.0, 3.0
    d[5, 0], d[5, 1], d[5, 2] = 4.0, 2.0, 1.0
    d[2, 0] = 200.0  # above 100 (also a mandatory neighbour)
    return d


SEEDS = [(1, 0), (0, 1), (2, 0), (0, 2), (2, 1), (1, 2), (3, 1), (1, 3), (3, 2), (2, 3),
         (4, 2), (2, 4), (4, 3), (3, 4), (5, 3), (3, 5), (5, 4), (4, 5)]


def test_hand_worked_no_existing_edges():
    new, ne = orc.proximity_select(_d(), 6, 0, 0, 1, 1, 16.0, [], [])
    # greedy: (5,2) suppresses (5,1); (4,1) suppresses (4,0); (5,0); (3,0); (4,0) is 20 > 16
    greedy = [(5, 2), (2, 5), (4, 1), (1, 4), (5, 0), (0, 5), (3, 0), (0, 3)]
    assert ne == 26
    assert [tuple(e) for e in new] == SEEDS + greedy


def test_hand_worked_existing_active_and_inactive_edges():
    new, ne = orc.proximity_select(_d(), 6, 0, 0, 1, 1, 16.0, [1], [0], ii_inac=[5],
                                   jj_inac=[2])
    # (1,0) exists: its seed pair is skipped in both directions; (5,2) inactive
    # suppresses itself and (5,1)
    seeds = SEEDS[2:]
    greedy = [(4, 1), (1, 4), (5, 0), (0, 5), (3, 0), (0, 3)]
    assert ne == 22
    assert [tuple(e) for e in new] == seeds + greedy


def test_max_factors_cut():
    new, ne = orc.proximity_select(_d(), 6, 0, 0, 1, 1, 16.0, [], [], max_factors=20)
    # 18 seed edges; (5,2) taken (18 <= 20), (5,1) suppressed, (4,1) taken
    # (20 <= 20), then 22 > 20 stops the greedy loop
    assert ne == 22
    assert [tuple(e) for e in new] == SEEDS + [(5, 2), (2, 5), (4, 1), (1, 4)]


def test_invariants_on_random_windows():
    rng = np.random.default_rng(0)
    for _ in range(20):
        t = int(rng.integers(4, 14))
        t0, t1 = int(rng.integers(0, t)), int(rng.integers(0, t))
        rad, nms = int(rng.integers(0, 3)), int(rng.integers(0, 3))
        d = rng.uniform(0, 30, (t - t0) * (t - t1)).astype(np.float32)
        ii = rng.integers(0, t, 5)
        jj = rng.integers(0, t, 5)
        new, ne = orc.proximity_select(d, t, t0, t1, rad, nms, 16.0, ii, jj)
        have = set(zip(ii.tolist(), jj.tolist()))
        got = [tuple(e) for e in new]
        assert len(got) == len(set(got)) and not (set(got) & have)
        for i, j in got:
            # every new edge is a neighbour edge or a candidate pair kept by the rules
            assert abs(i - j) <= rad + 1 or (j, i) in got or (j, i) in have
        picked = [(i, j) for i, j in got if i - j > rad + 1]
        for i, j in picked:
            k = (i - t0) * (t - t1) + (j - t1)
            assert t0 <= i < t and t1 <= j < t and d[k] <= 16.0


# ----------------------------------------------------- edge-state update ---
def _coded_rows(n, shape, base):
    # row e holds base + 100 e + (element index): shows which row went where
    k = int(np.prod(shape))
    return (base + 100.0 * np.arange(n)[:, None] + np.arange(k)[None, :]).reshape(
        (n,) + shape).astype(np.float32)


def test_oldest_mask_hand_worked():
    # ages 5 at edges 1, 2, 4: the two oldest are 1 and 2 (edge order among equals)
    np.testing.assert_array_equal(orc.oldest_mask([3, 5, 5, 1, 5, 0], 2), [0, 1, 1, 0, 0, 0])
    np.testing.assert_array_equal(orc.oldest_mask([3, 5, 5, 1, 5, 0], 4), [1, 1, 1, 0, 1, 0])
    np.testing.assert_array_equal(orc.oldest_mask([2, 7], 9), [1, 1])
    np.testing.assert_array_equal(orc.oldest_mask([2, 7], 0), [0, 0])


def test_store_and_remove_edges_hand_worked():
    # 6 edges, mask 1, 3, 4; the inactive list holds one edge and has room for
    # two more: 1 and 3 are stored, 4 is dropped; 0, 2, 5 close up in order
    ii, jj = [10, 11, 12, 13, 14, 15], [20, 21, 22, 23, 24, 25]
    age = [0, 1, 2, 3, 4, 5]
    nets, tg, wt = (_coded_rows(6, (3, 4), b) for b in (0.0, 1000.0, 2000.0))
    tin, win = _coded_rows(1, (2, 2), 5000.0), _coded_rows(1, (2, 2), 6000.0)
    tg, wt = tg[:, :2, :2].copy(), wt[:, :2, :2].copy()
    r = orc.store_and_remove_edges([0, 1, 0, 1, 1, 0], ii, jj, age, [7], [8], 3, nets, tg, wt,
                                   tin, win)
    assert r["n_kept"] == 3 and r["num_inac"] == 3
    np.testing.assert_array_equal(r["ii"], [10, 12, 15])
    np.testing.assert_array_equal(r["jj"], [20, 22, 25])
    np.testing.assert_array_equal(r["age"], [0, 2, 5])
    np.testing.assert_array_equal(r["nets"], nets[[0, 2, 5]])
    np.testing.assert_array_equal(r["target"], tg[[0, 2, 5]])
    np.testing.assert_array_equal(r["weight"], wt[[0, 2, 5]])
    np.testing.assert_array_equal(r["ii_inac"], [7, 11, 13])
    np.testing.assert_array_equal(r["jj_inac"], [8, 21, 23])
    np.testing.assert_array_equal(r["target_inac"], np.concatenate([tin, tg[[1, 3]]]))
    np.testing.assert_array_equal(r["weight_inac"], np.concatenate([win, wt[[1, 3]]]))


def test_store_and_remove_edges_chain_of_moves():
    # removing edge 0 shifts every other edge down by one: each destination row
    # is the source of the move before it
    nets = _coded_rows(5, (2, 3), 0.0)
    tw = _coded_rows(5, (2, 3), 500.0)
    r = orc.store_and_remove_edges([1, 0, 0, 0, 0], range(5), range(5), range(5), [], [], 0,
                                   nets, tw, tw + 1, np.zeros((0, 2, 3)), np.zeros((0, 2, 3)))
    assert r["n_kept"] == 4 and r["num_inac"] == 0  # no room: edge 0 is dropped
    np.testing.assert_array_equal(r["nets"], nets[1:])
    np.testing.assert_array_equal(r["target"], tw[1:])
    np.testing.assert_array_equal(r["weight"], tw[1:] + 1)
    np.testing.assert_array_equal(r["ii"], [1, 2, 3, 4])


def test_init_new_edges_hand_worked():
    nets = _coded_rows(4, (2, 3), 0.0)
    en = _coded_rows(5, (2, 3), 9000.0)
    w = _coded_rows(5, (2, 3), 7000.0)
    ii = [1, 2, 3, 0, 2]
    en2, w2 = orc.init_new_edges(nets, en, w, ii, 3, 2)
    np.testing.assert_array_equal(en2[:3], en[:3])      # untouched
    np.testing.assert_array_equal(en2[3], nets[0])      # ii[3] = 0
    np.testing.assert_array_equal(en2[4], nets[2])      # ii[4] = 2
    np.testing.assert_array_equal(w2[:3], w[:3])
    np.testing.assert_array_equal(w2[3:], 0.0)


def _kf_state(t, ne, ni, hw, seed=0, fdtype=np.float16):
    rng = np.random.default_rng(seed)
    return {
        "poses": _coded_rows(t, (7,), 0.0), "disps": _coded_rows(t, (hw,), 10000.0),
        "fmaps": rng.normal(size=(t, 4, hw)).astype(fdtype),
        "nets": _coded_rows(t, (3, hw), 20000.0), "inps": _coded_rows(t, (3, hw), 30000.0),
        "ii": rng.integers(0, t, ne), "jj": rng.integers(0, t, ne),
        "age": np.arange(ne), "ii_inac": rng.integers(0, t, ni), "jj_inac": rng.integers(0, t, ni),
        "edge_nets": _coded_rows(ne, (3, hw), 40000.0), "target": _coded_rows(ne, (2, hw), 5e4),
        "weight": _coded_rows(ne, (2, hw), 6e4), "target_inac": _coded_rows(ni, (2, hw), 7e4),
        "weight_inac": _coded_rows(ni, (2, hw), 8e4)}


def test_rm_keyframe_hand_worked():
    st = _kf_state(5, 6, 3, 4)
    st["ii"], st["jj"] = np.array([0, 2, 1, 3, 4, 2]), np.array([1, 3, 0, 4, 2, 1])
    st["ii_inac"], st["jj_inac"] = np.array([2, 4, 0]), np.array([0, 3, 1])
    r = orc.rm_keyframe(2, st)
    # keyframes 3, 4 move to 2, 3; row 4 keeps its old content
    for k in ("poses", "disps", "fmaps", "nets", "inps"):
        np.testing.assert_array_equal(r[k][:2], st[k][:2])
        np.testing.assert_array_equal(r[k][2:4], st[k][3:5])
        np.testing.assert_array_equal(r[k][4], st[k][4])
    # edges touching 2 (1, 4, 5) go; 3 -> 2, 4 -> 3
    np.testing.assert_array_equal(r["ii"], [0, 1, 2])
    np.testing.assert_array_equal(r["jj"], [1, 0, 3])
    np.testing.assert_array_equal(r["age"], [0, 2, 3])
    for k in ("edge_nets", "target", "weight"):
        np.testing.assert_array_equal(r[k][:3], st[k][[0, 2, 3]])
    # inactive: (2,0) goes; (4,3) -> (3,2); (0,1) stays
    np.testing.assert_array_equal(r["ii_inac"], [3, 0])
    np.testing.assert_array_equal(r["jj_inac"], [2, 1])
    for k in ("target_inac", "weight_inac"):
        np.testing.assert_array_equal(r[k][:2], st[k][[1, 2]])
    # out of range: nothing changes
    r = orc.rm_keyframe(5, st)
    np.testing.assert_array_equal(r["ii"], st["ii"])
    np.testing.assert_array_equal(r["nets"], st["nets"])
