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


# ------------------------------------------------------------------------------------------------ two-choice placement
def test_set2_hand_values():
    # 1 * 2654435761 >> 12 = 648055 (by hand: 2654435761 / 4096 = 648055.6), 648055 = 7 * 92579 + 2
    assert ref.wcache_set2(1, 7) == 2
    assert ref.wcache_set2(0, 5) == 0
    # rows near 2^31: the product needs 63 bits (a 32-bit product would wrap)
    assert ref.wcache_set2(2147483647, 1000) == 112 and ref.wcache_set2(2147483646, 4096) == 2320
    assert ref.wcache_set2(12345, 64) == 52


def test_step2_reduces_and_hand_example():
    g = np.random.default_rng(3)
    for _ in range(10):                                   # S = 1: the second set is the first
        W = int(g.choice([2, 4]))
        tag = np.full(W, -1)
        tag[:W // 2] = g.choice(50, W // 2, replace=False)
        idx = g.integers(-1, 52, (2, 20))
        a, b = ref.wcache_step(tag, [0], idx, 50, W), ref.wcache_step2(tag, [0], idx, 50, W)
        assert a["hits"] == b["hits"] and a["pinned"] == b["pinned"] and a["misses"] == b["misses"]
    # W = 1, S = 7: set2(1) = 2. Row 1 cached in its second set (line 2) hits there; row 8 (set 1) cached in set 1
    out = ref.wcache_step2([-1, 8, 1, -1, -1, -1, -1], [0] * 7, [[1, 8, 15, 1]], 20, 1)
    assert out["hits"] == 3 and out["pinned"] == {1, 2} and out["misses"] == [15]


def _serial2(tag, rr, idx, R, W, order_seed, plant=None):
    """The two-choice rule run one miss at a time in a random order (each miss: ticket in its first set, then in its
    second, then spill). plant: a deliberate mistake for the verifier to catch."""
    tag = np.array(tag, dtype=np.int64)
    S = tag.shape[0] // W
    m = ref.wcache_step2(tag, rr, idx, R, W)
    pinned, miss = m["pinned"], list(m["misses"])
    np.random.default_rng(order_seed).shuffle(miss)
    cnt, spills = np.zeros(S, int), 0
    for h in miss:
        placed = False
        sets = [h % S] if plant == "no_second" else [h % S, ref.wcache_set2(h, S)]
        if plant == "third_set":
            sets = [h % S, (ref.wcache_set2(h, S) + 1) % S]
        for st in sets:
            free = [st * W + (rr[st] + j) % W for j in range(W) if st * W + (rr[st] + j) % W not in pinned]
            tk = cnt[st]
            cnt[st] += 1
            if tk < len(free):
                tag[free[tk]] = h
                placed = True
                break
        spills += 0 if placed else 1
    if plant == "pinned" and pinned:
        tag[min(pinned)] = miss[0] if miss else 10 ** 6
    if plant == "spill":
        spills += 1
    adv = np.minimum(cnt, W) + (1 if plant == "rr" else 0)
    return tag, (np.asarray(rr) + adv) % W, spills


def _cases(seed, n):
    g = np.random.default_rng(seed)
    for _ in range(n):
        W = int(g.choice([1, 2, 4]))
        S = int(g.integers(2, 12))
        C = W * S
        R = int(g.integers(2 * C, 5 * C))
        tag = np.full(C, -1)
        rows = g.permutation(R)[:C]                        # a valid prior state: distinct rows in one of their sets
        for i, h in enumerate(rows):
            st = int(h % S) if g.random() < 0.6 else ref.wcache_set2(h, S)
            free = [st * W + w for w in range(W) if tag[st * W + w] < 0]
            if free and not np.isin(tag, h).any():
                tag[free[0]] = h
        rr = g.integers(0, W, S)
        idx = g.integers(-2, R + 2, (2, int(g.integers(4, 4 * C))))
        yield tag, rr, idx, R, W


def test_verify2_accepts_every_serial_order():
    n_overflow = 0
    for tag, rr, idx, R, W in _cases(5, 40):
        m = ref.wcache_step2(tag, rr, idx, R, W)
        for seed in range(4):
            t2, rr2, sp = _serial2(tag, rr, idx, R, W, seed)
            assert ref.wcache_verify2(m, tag, rr, t2, rr2, sp) == []
            n_overflow += sp > 0
    assert n_overflow > 10                                 # the cases exercise full sets


def test_verify2_catches_planted_mistakes():
    """A replaced pinned line, a miscounted spill or a wrong rr advance is caught whenever it changes the outcome. A
    missing second-set ticket or a row placed in a third set can leave a state that some valid order also leaves
    (e.g. every set full at W = 1), so those need only be caught in some of the cases."""
    for plant in ("no_second", "third_set", "pinned", "spill", "rr"):
        caught = changed = 0
        for tag, rr, idx, R, W in _cases(7, 40):
            m = ref.wcache_step2(tag, rr, idx, R, W)
            good = _serial2(tag, rr, idx, R, W, 0)
            bad = _serial2(tag, rr, idx, R, W, 0, plant=plant)
            if any(not np.array_equal(np.asarray(x), np.asarray(y)) for x, y in zip(good, bad)):
                changed += 1
                hit = ref.wcache_verify2(m, tag, rr, *bad) != []
                caught += hit
                if plant in ("pinned", "spill", "rr"):
                    assert hit, plant
        assert caught > 0 and (plant in ("pinned", "spill", "rr") or caught >= changed // 3), (plant, caught, changed)
