"""Host logic of the automatic-k sweep (emeans-cluster/src/auto.rs): seeds and
the choice of k, without a GPU."""

from emeans_amd import auto


def test_seed_for_wraps_like_u32():
    cfg = auto.AutoConfig(seed=0xFFFFFFF0)
    for salt, k, r in [(0, 0, 0), (3, 40, 3), (70000, 17, 5), (1 << 20, 1 << 20, 9)]:
        want = (cfg.seed + salt * 7919 + k * 131 + r * 1_000_003) % (1 << 32)
        assert auto.seed_for(cfg, salt, k, r) == want


def _s(k, sil, db, br):
    return auto.KScore(k, k, sil, 0.0, db, 0.0, br, 0.0)


def test_select_level1_smallest_k_within_tolerance():
    scores = [_s(2, 0.30, 1.0, 0.1), _s(3, 0.40, 1.0, 0.1), _s(4, 0.41, 1.0, 0.1)]
    cfg = auto.AutoConfig()
    assert auto.select(scores, cfg, False) == 2  # argmax at tolerance 0
    cfg.level1_tolerance = 0.05  # 0.40 >= 0.41 - 0.0205
    assert auto.select(scores, cfg, False) == 1


def test_select_level2_prefers_browsable_then_smaller_k():
    cfg = auto.AutoConfig()  # Davies-Bouldin (lower is better), tolerance 0.05
    scores = [_s(2, 0, 1.00, 0.5), _s(3, 0, 1.02, 0.9), _s(4, 0, 1.04, 0.9), _s(5, 0, 1.30, 1.0)]
    # candidates: -db >= -1.0 - 0.05: k = 2, 3, 4; most browsable 0.9, smaller k -> k = 3
    assert auto.select(scores, cfg, True) == 1


def test_browsable_fraction():
    cfg = auto.AutoConfig(min_cluster_size=20, max_cluster_size=200)
    assert auto.browsable([10, 20, 200, 201, 0], cfg) == (20 + 200) / 431
