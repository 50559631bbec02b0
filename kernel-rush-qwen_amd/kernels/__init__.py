"""Drop-in replacement for the reference engine's `kernels` package, decode-matmul path only.

The reference engine imports every kernel module from one package, `kernels`, with engine/ on
sys.path (engine/engine.py:49-61): the modules this package replaces - fp8, gemv, fused_gemv, mlp
(plus lmhead, packfile) - and others that stay the engine's own (flash_prefill, fused_attn, pdl,
mega, prefill_mlp, spec, ops, rmsnorm). So that both resolve, this package's search path is
extended after its own directory:

  - with every other `kernels` directory found on sys.path (pkgutil.extend_path), so putting this
    package's parent directory ahead of engine/ on sys.path is enough;
  - with the directory named by the environment variable KRQ_ENGINE_KERNELS (the engine's
    engine/kernels directory), for callers that do not keep engine/ on sys.path.

A module found here always wins; any other name is imported from the engine's directory, and
the engine's modules that import `from kernels import pdl` or `from kernels.ops import ...` get
their own files. The compute of the replaced modules runs in libkrq.so (hand-written gfx950 HIP
kernels behind the C ABI of include/krq.h); they keep the reference's Python signatures, output
contracts and exception types.
"""

import os
import pkgutil

__path__ = pkgutil.extend_path(__path__, __name__)

_engine_dir = os.environ.get("KRQ_ENGINE_KERNELS")
if _engine_dir:
    _engine_dir = os.path.abspath(_engine_dir)
    if not os.path.isdir(_engine_dir):
        raise ImportError(f"KRQ_ENGINE_KERNELS={_engine_dir!r} is not a directory")
    if _engine_dir not in [os.path.abspath(p) for p in __path__]:
        __path__.append(_engine_dir)

# the modules of the reference's package that this one replaces (the rest resolve from the engine)
REPLACED = ("fp8", "gemv", "fused_gemv", "mlp")
