"""On-disk pre-packed FP8 weights: quantize once, reload bit-exactly, check every tensor.

The reference re-quantizes its BF16 weights at every load (engine/engine.py:496-501). This format
stores what the quantizers produce - the row-major e4m3 bytes `w8` exactly as the reference's
quantizer lays them out, the fp32 scale (per tensor or per output row) and, optionally, the tiled
copy the GEMVs stream - in a safetensors file, with a SHA-256 digest per weight over its canonical
bytes (row-major w8, then the scale's little-endian fp32 bytes), so the packing contract can be
checked offline against any other producer of the same bytes.

File layout (safetensors):
  tensors    "<name>.w8"     uint8 [N, K]      row-major e4m3 codes
             "<name>.scale"  float32 [] or [N]
             "<name>.tiled"  uint8 [N*K]       optional; the tiled layout of include/krq.h
  metadata   "format" = "krq-fp8", "version" = "1",
             "<name>.sha256" = digest of w8 || scale, "<name>.tiled.sha256" when stored.
Loading verifies the digests (ValueError on any mismatch) and, when no tiled copy is stored and
one is wanted, rebuilds it on the device with krq_pack_fp8.
"""

import hashlib
import json

import torch

from . import _lib as L
from .fp8 import FP8Weight

FORMAT, VERSION = "krq-fp8", "1"


def _digest(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def _cpu_u8(t):
    return t.detach().to("cpu").contiguous().view(torch.uint8)


def save_fp8(path, weights, meta=None, tiled=False):
    """Write {name: FP8Weight} to `path`. tiled=True also stores the tiled copies (those present).
    `meta` (JSON-serializable) is kept under "user"."""
    from safetensors.torch import save_file
    tensors, md = {}, {"format": FORMAT, "version": VERSION}
    if meta is not None:
        md["user"] = json.dumps(meta)
    for name, q in weights.items():
        if "." in name:
            raise ValueError(f"weight name {name!r} must not contain '.'")
        w8, scale = q[0], q[1]
        if w8.dtype != torch.float8_e4m3fn or w8.dim() != 2:
            raise ValueError(f"{name}: expected a float8_e4m3fn [N, K] matrix")
        u8 = _cpu_u8(w8)
        sc = scale.detach().to("cpu", torch.float32).contiguous()
        if sc.numel() not in (1, w8.shape[0]):
            raise ValueError(f"{name}: scale must be per tensor or per row")
        tensors[f"{name}.w8"] = u8
        tensors[f"{name}.scale"] = sc
        md[f"{name}.sha256"] = _digest(u8, sc)
        t = getattr(q, "tiled", None)
        if tiled and t is not None:
            tu8 = _cpu_u8(t).reshape(-1)
            tensors[f"{name}.tiled"] = tu8
            md[f"{name}.tiled.sha256"] = _digest(tu8)
    save_file(tensors, path, metadata=md)


def read_meta(path):
    """The user metadata dict stored with the file (or None)."""
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        md = f.metadata() or {}
    return json.loads(md["user"]) if "user" in md else None


def load_fp8(path, device="cpu", tiled=True, verify=True):
    """Read {name: FP8Weight} from `path` onto `device`. Digests are checked (verify=True). With
    tiled=True each weight gets its tiled copy: the stored one, or one rebuilt on a ROCm device."""
    from safetensors import safe_open
    out = {}
    with safe_open(path, framework="pt") as f:
        md = f.metadata() or {}
        if md.get("format") != FORMAT or md.get("version") != VERSION:
            raise ValueError(f"{path}: not a {FORMAT} v{VERSION} file (format={md.get('format')!r}, "
                             f"version={md.get('version')!r})")
        names = sorted({k.rsplit(".", 1)[0] for k in f.keys() if k.endswith(".w8")})
        for name in names:
            u8 = f.get_tensor(f"{name}.w8")
            sc = f.get_tensor(f"{name}.scale")
            if verify and _digest(u8, sc) != md.get(f"{name}.sha256"):
                raise ValueError(f"{path}: {name} does not match its SHA-256 digest")
            t = None
            if tiled and f"{name}.tiled" in f.keys():
                t = f.get_tensor(f"{name}.tiled")
                if verify and _digest(t) != md.get(f"{name}.tiled.sha256"):
                    raise ValueError(f"{path}: {name}.tiled does not match its SHA-256 digest")
                t = t.to(device)
            w8 = u8.view(torch.float8_e4m3fn).to(device)
            sc = sc.to(device)
            N, K = w8.shape
            if tiled and t is None and N % 16 == 0 and K % 64 == 0:
                L.require_device(w8)
                t = torch.empty((N * K,), device=w8.device, dtype=torch.uint8)
                L.call("krq_pack_fp8", L.ptr(w8), N, K, L.ptr(t), L.stream(w8))
            out[name] = FP8Weight(w8, sc, t if tiled else None)
    return out
