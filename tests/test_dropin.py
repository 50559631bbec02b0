"""The drop-in boundary as the reference engine sees it (CPU, no GPU needed).

1. Import resolution: engine/engine.py:49-61 imports all of its kernel modules from one package,
   `kernels`. With this package's directory ahead of the engine's on sys.path (or the engine's
   kernels directory named by KRQ_ENGINE_KERNELS), every one of those imports must succeed: the
   replaced modules (fp8, gemv, fused_gemv, mlp) from here, the others (flash_prefill, fused_attn,
   pdl, mega, prefill_mlp, spec, ops) from the engine, including the engine modules' own
   `from kernels import pdl` / `from kernels.ops import ...`. The engine side is a temporary
   directory of stub modules written here (no reference code); its copies of the replaced modules
   raise on import, so resolving one of them there fails the test.
2. Signatures: every public function and constructor of the replaced modules accepts every call
   the reference's signature accepts (tests/golden/reference_signatures.json, transcribed from the
   reference's files), and the module / instance attributes the engine reads exist.
"""

import inspect
import json
import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "kernel-rush-qwen_amd")
SIGS = os.path.join(ROOT, "tests", "golden", "reference_signatures.json")

# the import block of engine/engine.py:49-61, verbatim in meaning
ENGINE_IMPORTS = textwrap.dedent("""
    from kernels.flash_prefill import flash_prefill
    from kernels.fused_attn import FusedDecodeAttention
    from kernels import pdl
    from kernels.mega import MegaDecode
    from kernels.mlp import PersistentMLP
    from kernels.prefill_mlp import gu_swiglu
    from kernels import fp8
    from kernels.fp8 import ActScale, SharedScale, linear_fp8, quantize_weight
    from kernels.fused_gemv import FusedLayerBuffers, gemv_fused, gemv_swiglu_fused
    from kernels.gemv import gemv, gemv_m1, gemv_m1_swiglu, gemv_rows, gemv_swiglu, gemv_tma
    from kernels.spec import accept as spec_accept, draft as spec_draft
    from kernels.ops import (DecodeAttention, add_rmsnorm, qk_norm_rope_cache,
                             qk_norm_rope_cache_prefill, silu_mul)
""")

STUBS = {
    "__init__.py": "",
    "pdl.py": "def enable(*a, **k): return False\ndef pdl_launch(): pass\ndef pdl_wait(): pass\n",
    "ops.py": ("from kernels import pdl\n_DOT_F32 = False\n"
               "class DecodeAttention: pass\n"
               "def _load_rows(*a): pass\ndef add_rmsnorm(*a): pass\ndef qk_norm_rope_cache(*a): pass\n"
               "def qk_norm_rope_cache_prefill(*a): pass\ndef silu_mul(*a): pass\n"),
    "fused_attn.py": ("from kernels import pdl\nfrom kernels.ops import _DOT_F32, DecodeAttention, _load_rows\n"
                      "from kernels.pdl import pdl_launch, pdl_wait\nclass FusedDecodeAttention: pass\n"
                      "def _norm_rope_half(*a): pass\n"),
    "flash_prefill.py": "def flash_prefill(*a): pass\n",
    "mega.py": "from kernels.fused_attn import _norm_rope_half\nclass MegaDecode: pass\n",
    "prefill_mlp.py": "def gu_swiglu(*a): pass\n",
    "spec.py": "def accept(*a): pass\ndef draft(*a): pass\n",
}
REPLACED = ("fp8", "gemv", "fused_gemv", "mlp")


def _engine_tree(tmp_path):
    kdir = tmp_path / "engine" / "kernels"
    kdir.mkdir(parents=True)
    for name, src in STUBS.items():
        (kdir / name).write_text(src)
    for name in REPLACED:
        (kdir / f"{name}.py").write_text(f"raise ImportError('the engine stub of {name} was imported')\n")
    return kdir


CHECK = ENGINE_IMPORTS + textwrap.dedent("""
    import kernels, os, sys
    here = os.path.realpath(sys.argv[1])
    there = os.path.realpath(sys.argv[2])
    for name in ("fp8", "gemv", "fused_gemv", "mlp"):
        f = os.path.realpath(sys.modules["kernels." + name].__file__)
        assert f.startswith(here), (name, f)
    for name in ("flash_prefill", "fused_attn", "pdl", "mega", "prefill_mlp", "spec", "ops"):
        f = os.path.realpath(sys.modules["kernels." + name].__file__)
        assert f.startswith(there), (name, f)
    print("resolved", len(kernels.__path__), "dirs")
""")


def _run(path_entries, env_extra, kdir):
    env = dict(os.environ)
    env.pop("KRQ_ENGINE_KERNELS", None)
    env.update(env_extra)
    env["PYTHONPATH"] = os.pathsep.join(path_entries)
    r = subprocess.run([sys.executable, "-c", CHECK, os.path.join(PKG, "kernels"), str(kdir)],
                       capture_output=True, text=True, env=env, cwd=str(kdir.parent.parent), timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "resolved" in r.stdout


def test_engine_imports_resolve_with_package_first_on_sys_path(tmp_path):
    kdir = _engine_tree(tmp_path)
    _run([PKG, str(kdir.parent)], {}, kdir)


def test_engine_imports_resolve_with_env_variable(tmp_path):
    kdir = _engine_tree(tmp_path)
    _run([PKG], {"KRQ_ENGINE_KERNELS": str(kdir)}, kdir)


def test_bad_env_variable_is_an_import_error(tmp_path):
    env = dict(os.environ, KRQ_ENGINE_KERNELS=str(tmp_path / "missing"), PYTHONPATH=PKG)
    r = subprocess.run([sys.executable, "-c", "import kernels"], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode != 0 and "KRQ_ENGINE_KERNELS" in r.stderr


def _resolve(qual):
    import importlib
    mod, *rest = qual.split(".")
    obj = importlib.import_module(f"kernels.{mod}")
    for part in rest:
        obj = getattr(obj, part)
    return obj


def _compatible(ours, ref):
    """True if every call the reference parameter list accepts is accepted by `ours` with the same
    meaning: the reference's parameters in order, same names and kinds, same defaults where the
    reference has one (a default where the reference requires the argument is allowed); any
    extra parameter of ours comes after them and has a default."""
    params = list(ours.parameters.values())
    if len(params) < len(ref):
        return f"{len(params)} parameters, reference has {len(ref)}"
    for p, (name, kind, default) in zip(params, ref):
        if p.name != name or p.kind.name != kind:
            return f"parameter {p.name} ({p.kind.name}) where the reference has {name} ({kind})"
        if default is not None and (p.default is inspect.Parameter.empty or repr(p.default) != default):
            return f"{name} defaults to {p.default!r}, reference {default}"
    for p in params[len(ref):]:
        if p.default is inspect.Parameter.empty and p.kind not in (p.VAR_POSITIONAL, p.VAR_KEYWORD):
            return f"extra parameter {p.name} has no default"
    return None


def test_signatures_match_the_reference():
    spec = json.load(open(SIGS))
    bad = []
    for qual, ref in spec["functions"].items():
        why = _compatible(inspect.signature(_resolve(qual)), ref)
        if why:
            bad.append(f"{qual}: {why}")
    for mod, names in spec["attributes"].items():
        m = _resolve(mod)
        bad += [f"{mod}.{n} missing" for n in names if not hasattr(m, n)]
    assert not bad, "\n".join(bad)


def test_instance_attributes_the_engine_reads():
    import torch
    from kernels import fp8
    from kernels.fused_gemv import FusedLayerBuffers
    from kernels.mlp import PersistentMLP
    spec = json.load(open(SIGS))["instance_attributes"]
    objs = {
        "fused_gemv.FusedLayerBuffers": FusedLayerBuffers(1, 2560, 151936, "cpu"),
        "mlp.PersistentMLP": PersistentMLP(1, 2560, 9728, "cpu", 132),
        "fp8.SharedScale": fp8.SharedScale(torch.ones(1), torch.ones(())),
    }
    for qual, names in spec.items():
        if qual not in objs:
            continue
        missing = [n for n in names if not hasattr(objs[qual], n)]
        assert not missing, (qual, missing)
    assert fp8.FP8_MAX == 448.0
