"""TreeSparseMetadataCache keying (host logic; the builds are stubs, no GPU)."""

import torch

import eagle_tree_sparse_bridge as bridge


def _cache_and_counter(capacity=4):
    cache = bridge.TreeSparseMetadataCache(capacity)
    built = []

    def build(tag):
        def f():
            built.append(tag)
            return f"meta-{tag}-{len(built)}"
        return f

    return cache, built, build


def test_same_tensor_and_geometry_hits():
    cache, built, build = _cache_and_counter()
    m = torch.zeros(1, 1, 8, 40)
    a = cache.get(m, (32, 8, 16, 64, 0), build("a"))
    b = cache.get(m, (32, 8, 16, 64, 0), build("b"))
    assert a == b and built == ["a"] and cache.hits == 1 and cache.builds == 1


def test_in_place_write_rebuilds():
    cache, built, build = _cache_and_counter()
    m = torch.zeros(1, 1, 8, 40)
    cache.get(m, (32,), build("a"))
    m[0, 0, 0, 0] = float("-inf")  # bumps the version counter
    cache.get(m, (32,), build("b"))
    assert built == ["a", "b"]


def test_geometry_and_views_are_part_of_the_key():
    cache, built, build = _cache_and_counter()
    m = torch.zeros(2, 1, 8, 40)
    cache.get(m, (32, 16, 64, 0), build("a"))
    cache.get(m, (32, 16, 64, 1), build("b"))     # another batch index
    cache.get(m, (32, 16, 32, 0), build("c"))     # another BLOCK_N
    cache.get(m[1:], (32, 16, 64, 0), build("d"))  # another view (pointer and shape)
    assert built == ["a", "b", "c", "d"]


def test_capacity_evicts_least_recently_used_and_keeps_sources_alive():
    cache, built, build = _cache_and_counter(capacity=2)
    t1, t2, t3 = torch.zeros(4), torch.zeros(4), torch.zeros(4)
    cache.get(t1, (), build("1"))
    cache.get(t2, (), build("2"))
    cache.get(t1, (), build("x"))  # hit: t1 becomes most recent
    cache.get(t3, (), build("3"))  # evicts t2
    cache.get(t1, (), build("y"))  # still cached
    cache.get(t2, (), build("2b"))
    assert built == ["1", "2", "3", "2b"]
    assert all(e[0] is not None for e in cache._entries.values())


def test_capacity_must_be_positive():
    import pytest

    with pytest.raises(ValueError):
        bridge.TreeSparseMetadataCache(0)
