"""Properties of the seeded generators (xlog_amd/csrc/datagen.c)."""
import numpy as np

from xlog_amd import datagen, pack


def test_random_digraph_distinct_no_self_loops_deterministic():
    s1, d1 = datagen.random_digraph(1000, 5000, datagen.seed_for(1))
    s2, d2 = datagen.random_digraph(1000, 5000, datagen.seed_for(1))
    assert np.array_equal(s1, s2) and np.array_equal(d1, d2)
    assert not np.any(s1 == d1)
    assert len(np.unique(pack(s1, d1))) == 5000
    assert s1.max() < 1000 and d1.max() < 1000
    s3, _ = datagen.random_digraph(1000, 5000, datagen.seed_for(1) + 1)
    assert not np.array_equal(s1, s3)


def test_lcg_matches_reference_recurrence():
    """s <- s * 6364136223846793005 + 1 (crates/xlog-gpu/benches/logic_bench.rs:48-62)."""
    src, dst = datagen.ref_random_graph(1000, 4, 123)
    s = 123
    exp = []
    for _ in range(8):
        s = (s * 6364136223846793005 + 1) % (1 << 64)
        exp.append(s % 1000)
    assert src.tolist() == exp[0::2] and dst.tolist() == exp[1::2]


def test_dup_tuples_exact_duplicate_fraction():
    n = 1 << 18
    k = datagen.dup_tuples(n, datagen.seed_for(3))
    assert len(np.unique(k)) == n - (n * 3) // 10  # fresh values are 64-bit uniform: no collisions at this size


def test_zipf_join_skew_and_keys():
    r_a, r_b, s_b, s_c = datagen.zipf_join(1 << 18, 1 << 18, 1 << 12, 1.1, datagen.seed_for(2))
    keys = [datagen.key_of_rank(i, datagen.seed_for(2)) for i in range(1 << 12)]
    assert len(set(keys)) == 1 << 12
    assert set(np.unique(s_b).tolist()) <= set(keys)
    vals, cnt = np.unique(r_b, return_counts=True)
    top = vals[np.argmax(cnt)]
    assert top == keys[0]
    # rank-1 probability of Zipf(1.1) over 4096 keys
    h = sum((k + 1) ** -1.1 for k in range(1 << 12))
    assert abs(cnt.max() / len(r_b) - 1 / h) < 0.01


def test_andersen_relations_distinct():
    f = datagen.andersen(5000, 20000, 1.5, datagen.seed_for(5))
    assert [len(f[k][0]) for k in ("assign", "addressOf", "load", "store")] == [8000, 4000, 4000, 4000]
    for k in f:
        v, w = f[k]
        assert not np.any(v == w)
        assert len(np.unique(pack(v, w))) == len(v)
        assert v.max() < 5000 and w.max() < 5000
