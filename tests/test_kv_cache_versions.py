"""Cache versions on the CPU: the decoder keys each layer's block images on (id(K), id(V), K.generation,
V.generation, length). Python reuses the id() of a freed object, so the generations must never repeat across caches:
every new cache, every append and every touch() takes a value that no cache has held before."""
import gc

import torch

from opendecider_amd.kv_cache import Int8KVCache, StateKV


def _image_key(k, v):
    return (id(k), id(v), k.generation, v.generation, k.length)


def test_fresh_caches_never_repeat_an_image_key():
    """The serving pattern that used to collide: a fresh cache pair per request, set to the same length and freed
    after use. Every request's key differs from every earlier one, id() reuse included."""
    seen = set()
    for _ in range(200):
        k = Int8KVCache(1, 2, 8, 16, "cpu")
        v = Int8KVCache(1, 2, 8, 16, "cpu")
        k.length = v.length = 16
        k.touch()
        v.touch()
        key = _image_key(k, v)
        assert key not in seen
        seen.add(key)
        del k, v
        gc.collect()


def test_state_kv_views_and_touch_take_new_generations():
    st = StateKV(3, 2, 2, 8, 16, "cpu")
    gens = [c.generation for pair in st for c in pair]
    assert len(set(gens)) == len(gens)
    k, _ = st[0]
    before = k.generation
    k.touch()
    assert k.generation != before and k.generation not in gens


def test_append_moves_the_generation():
    c = Int8KVCache.from_tensors(torch.zeros(1, 1, 4, 8, dtype=torch.int8), torch.zeros(1, 1, 4))
    g0 = c.generation
    c.touch()
    assert c.generation > g0
