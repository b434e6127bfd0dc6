"""Loader of the C++ attention backend extension (module ``sgl_backend``).

The extension holds HipAttnBackend, MHAKVCache, RMSNorm, RotaryEmbedding and
AttentionLayer — the reference's BaseAttnBackend contract and the layer
around it (include/sglang/attention/backend.h:16-41,
src/layers/attention_layer.cc:17-51) — over libsgl_attn.so. It is built
in-tree by build.py; loading fails loudly when it is missing.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import sysconfig
from pathlib import Path

_PKG_DIR = Path(__file__).resolve().parent
_MOD = None


def path() -> Path:
    return _PKG_DIR / ("sgl_backend" + sysconfig.get_config_var("EXT_SUFFIX"))


def load():
    """Import and return the built extension module."""
    global _MOD
    if _MOD is None:
        p = path()
        if not p.exists():
            raise RuntimeError(f"{p} is not built: run `python sglang.cpp_amd/build.py` "
                               "(or __graft_entry__.build())")
        import torch  # noqa: F401  (loads libtorch / libc10_hip first)
        loader = importlib.machinery.ExtensionFileLoader("sgl_backend", str(p))
        spec = importlib.util.spec_from_file_location("sgl_backend", p, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _MOD = mod
    return _MOD
