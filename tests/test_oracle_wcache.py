"""Pins of the oracle's W-way row cache step: hand-worked W = 2 examples and a sequential simulation of the ticketed
placement (each miss takes the next ticket of its set and the ticket-th unpinned way from rr) under random miss
orders, whose order-independent outputs must equal the model's. CPU only."""
import numpy as np

from oracle import spmla_ref as ref


def test_wcache_hand_examples():
    # C = 4, W = 2: set 0 = lines 0, 1 (row 4, empty); set 1 = lines 2, 3 (rows 3, 5); rr = [1, 0]
    out = ref.wcache_step([4, -1, 3, 5], [1, 0], [[4, 6, 8, 3, 7, 9, 11, -1, 4]], 20, 2)
    assert out["hits"] == 3 and out["pinned"] == {0, 2} and out["misses"] == [6, 7, 8, 9, 11]
    assert out["placed"] == {0: [1], 1: [3]} and out["spills"] == 3
    assert list(out["rr_next"]) == [1, 0] and out["content"] == {}
    out = ref.wcache_step([-1, -1, -1, -1], [0, 0], [[0, 1, 2, 2]], 10, 2)
    assert out["hits"] == 0 and out["misses"] == [0, 1, 2] and out["spills"] == 0
    assert out["placed"] == {0: [0, 1], 1: [2]} and list(out["rr_next"]) == [0, 1]
    assert out["content"] == {0: [0, 2], 1: [-1, 1]}


def _sequential(tag, rr, idx, R, W, order_seed):
    tag = np.array(tag, dtype=np.int64)
    C = tag.shape[0]
    S = C // W
    pinned, miss = set(), []
    for h in np.asarray(idx).reshape(-1):
        if 0 <= h < R:
            st = h % S
            w = [st * W + j for j in range(W) if tag[st * W + j] == h]
            if w:
                pinned.add(w[0])
            elif h not in miss:
                miss.append(int(h))
    np.random.default_rng(order_seed).shuffle(miss)
    cnt, spills, changed = np.zeros(S, int), 0, set()
    for h in miss:
        st = h % S
        free = [st * W + (rr[st] + j) % W for j in range(W) if st * W + (rr[st] + j) % W not in pinned]
        tk = cnt[st]
        cnt[st] += 1
        if tk < len(free):
            tag[free[tk]] = h
            changed.add(free[tk])
        else:
            spills += 1
    rr2 = (np.asarray(rr) + np.minimum(cnt, W)) % W
    return tag, rr2, spills, changed


def test_wcache_model_vs_sequential_orders():
    g = np.random.default_rng(0)
    for trial in range(20):
        W = int(g.choice([2, 4, 8]))
        C = W * int(g.integers(2, 40))
        R = int(g.integers(C, 6 * C))
        tag = np.full(C, -1)
        for st in range(C // W):                     # a valid prior state: distinct rows of the right set
            rows = [r for r in range(st, R, C // W)]
            g.shuffle(rows)
            k = int(g.integers(0, W + 1))
            tag[st * W:st * W + k] = rows[:k]
        rr = g.integers(0, W, C // W)
        idx = g.integers(-2, R + 2, (3, int(g.integers(5, 3 * C))))
        m = ref.wcache_step(tag, rr, idx, R, W)
        for seed in range(3):
            t2, rr2, spills, changed = _sequential(tag, rr, idx, R, W, seed)
            assert spills == m["spills"]
            assert np.array_equal(rr2, m["rr_next"])
            assert changed == {l for v in m["placed"].values() for l in v}
            assert all(t2[l] == tag[l] for l in m["pinned"])
            for st, want in m["content"].items():
                assert sorted(t2[st * W:(st + 1) * W].tolist()) == want
