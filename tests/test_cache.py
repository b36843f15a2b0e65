"""Keys of the prepared-launch cache (host logic only)."""

import torch

from torch_einshard import _cache


def test_key_depends_on_geometry_and_arguments():
    x = torch.empty(4, 6)
    base = _cache.call_key("einshard", (x,), None, None, "a b -> b a", None, None)
    assert base is not None
    assert _cache.call_key("einshard", (torch.empty(4, 6),), None, None, "a b -> b a", None, None) == base
    assert _cache.call_key("einshard", (x.t().contiguous().t(),), None, None, "a b -> b a", None, None) != base
    assert _cache.call_key("einshard", (x.double(),), None, None, "a b -> b a", None, None) != base
    assert _cache.call_key("einshard", (x,), None, None, "a b -> a b", None, None) != base
    assert _cache.call_key("einshard", (x,), None, None, "a b -> b a", {"a": 4}, None) != base
    # fill 1 and fill 1.0 convert alike but are kept apart
    k1 = _cache.call_key("einwindow", (x,), None, None, "a b -> a k b", {"a": "k"}, {"a": 1}, "constant", 1, None)
    k2 = _cache.call_key("einwindow", (x,), None, None, "a b -> a k b", {"a": "k"}, {"a": 1}, "constant", 1.0, None)
    assert k1 != k2


def test_calls_that_must_take_the_full_path_have_no_key():
    x = torch.empty(3)
    assert _cache.call_key("einshard", (x,), object(), None, "a -> a", None, None) is None  # mesh
    assert _cache.call_key("einshard", (x,), None, {"x": 1}, "a -> a", None, None) is None  # shapes
    assert _cache.call_key("einshard", ([1, 2, 3],), None, None, "a -> a", None, None) is None
    assert _cache.call_key("einshard", (torch.nn.Parameter(x),), None, None, "a -> a", None, None) is None
    assert _cache.call_key("einwindow", (x,), None, None, "a -> a k", {"a": "k"}, {"a": 1}, "constant", x, None) is None


def test_cache_is_bounded():
    _cache.clear()
    for i in range(_cache._LIMIT + 5):
        _cache.remember(("k", i), i)
    assert len(_cache._entries) <= _cache._LIMIT
    _cache.clear()
