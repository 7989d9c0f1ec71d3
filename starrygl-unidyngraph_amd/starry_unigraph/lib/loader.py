"""Loader of the native sampler module (mirror of lib/loader.py:7-9 in the reference)."""
from __future__ import annotations

import importlib
from functools import lru_cache


@lru_cache(maxsize=1)
def load_bts_sampler_module():
    """Returns ``starry_unigraph.lib.libstarrygl_sampler`` after checking that the
    HIP library loads and a GPU is present (raises otherwise, like the reference
    raises when its extension is missing)."""
    mod = importlib.import_module("starry_unigraph.lib.libstarrygl_sampler")
    from starry_unigraph.lib import _capi
    _capi.lib()
    _capi.require_gpu()
    return mod
