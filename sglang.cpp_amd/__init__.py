"""MI355X-native attention hot path of sglang.cpp (gfx950 HIP kernels).

The directory name is not a Python identifier; load it with
``load_package()`` from ``__graft_entry__`` (registered as
``sglang_cpp_amd``). Submodules:
  capi       ctypes binding of libsgl_attn.so (include/sgl_attn.h)
  workloads  seeded synthetic inputs for the benchmark configurations
  backend    loader of the C++ attention backend extension (sgl_backend)
  build      in-tree build of the HIP library and the C++ backend
"""
from . import backend, capi, workloads  # noqa: F401

__all__ = ["backend", "capi", "workloads"]
