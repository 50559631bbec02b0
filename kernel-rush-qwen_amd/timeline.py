"""Per-block timeline of the decode step's FP8 GEMV launches (M = 1 and M = 16 by default, any of 1,
16 and 32 with --m), read from the
timeline build of the library, whose GEMV kernel stamps the wall clock (100 MHz) per block at
  t0  entry,
  t1  activation slice ready (bf16 kinds: the activation wave's, or the whole block's, prologue
      done) or, for e4m3 activations, the step ring issued,
  t2  main loop done (the last step's matrix-core product),
  t3  outputs issued,
and the compute unit each block ran on (__smid: XCD, shader engine, CU).

    python kernel-rush-qwen_amd/build_lib.py --timeline     # on the build host: libkrq_timeline.so
    python kernel-rush-qwen_amd/timeline.py [--m 1,16,32] [--json PATH]    # on the GPU

Each projection runs the way bench.py's kernel table runs it (a graph of 72 launches cycling 36
layers' weights, hipEvents around each replay); the stamps are those of the graph's last launch.
Per projection it prints the graph-timed microseconds per launch, the blocks' span (first entry
to last outputs), the time per launch outside that span (launch and completion overhead plus
the gap to the next launch), percentiles over blocks of each stamp from the first entry, and
the blocks' outputs time (t3, median) grouped by how many of the launch's blocks shared their
compute unit.
"""

import argparse
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for _p in (ROOT, HERE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

LIB = os.path.join(HERE, "kernels", "libkrq_timeline.so")
SLOTS = 8 * 65536  # slots held by the timeline build (8 per block: t0..t3, compute unit)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--json", default=None, help="also write the summary here")
    ap.add_argument("--reps", type=int, default=72, help="launches per graph")
    ap.add_argument("--m", default="1,16", help="comma-separated rows per launch, each 1, 16 or 32 "
                    "(above one row: per-token tiled e4m3 rows, as bench.py's kernel table)")
    args = ap.parse_args()
    ms = [int(v) for v in args.m.split(",")]
    if not ms or any(v not in (1, 16, 32) for v in ms):
        sys.exit("timeline.py: --m takes 1, 16 and 32")
    if not os.path.exists(LIB):
        sys.exit(f"timeline.py: {LIB} is missing; build it first: python kernel-rush-qwen_amd/build_lib.py "
                 "--timeline")

    import numpy as np
    import torch

    from kernels import _lib as L
    L.LIB_PATH = LIB  # before the first load: every wrapper below then runs the timeline build
    lib = L.lib()
    lib.krq_timeline_read.restype = ctypes.c_int
    lib.krq_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    lib.krq_timeline_clock_khz.restype = ctypes.c_int
    import bench
    from kernels import fp8

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    khz = lib.krq_timeline_clock_khz()
    if khz <= 0:
        sys.exit("timeline.py: no wall-clock rate from the device")
    buf = np.zeros(SLOTS, dtype=np.uint64)

    def stamps():
        torch.cuda.synchronize()
        if lib.krq_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
            raise RuntimeError("krq_timeline_read failed")
        return buf.reshape(-1, 8).astype(np.int64)

    layers = bench.make_layers(torch, fp8, dev, bench.LAYERS)
    modes = {"partial": L.OUT_PARTIAL, "swiglu": L.OUT_SWIGLU, "bf16": L.OUT_BF16}
    out = {"clock_khz": khz, "reps": args.reps, "layers": bench.LAYERS, "launches": []}
    pct = (50, 90, 100)
    print(f"[timeline] wall clock {khz} kHz; graph of {args.reps} launches cycling {bench.LAYERS} layers; "
          f"stamps (us from the first block's entry) p50/p90/max over blocks", flush=True)
    print(f"  {'launch':<12} {'blocks':>6} {'us/launch':>9} {'span':>6} {'outside':>7} | {'t0 (entry)':>17} | "
          f"{'t1 (act ready)':>17} | {'t2 (loop done)':>17} | {'t3 (outputs)':>17}", flush=True)
    for M in ms:
        xs = bench.make_inputs(torch, dev, M)
        for name, N, K, split, mode in bench.PROJ:
            x, m = xs[name], modes[mode]
            if M == 1:
                o = fp8.gemv_fp8_bf16_launch(x, layers[0][name], split, m, None, L.ALGO_AUTO)

                def fn(i, x=x, name=name, split=split, m=m, o=o):
                    return fp8.gemv_fp8_bf16_launch(x, layers[i % len(layers)][name], split, m, None,
                                                    L.ALGO_AUTO, out=o)
            else:
                x8, sc = fp8.quant_rows_tiled(x)
                o = fp8.gemv_fp8_tiled_launch(x8, sc, layers[0][name], M, split, m)

                def fn(i, x8=x8, sc=sc, name=name, split=split, m=m, o=o):
                    return fp8.gemv_fp8_tiled_launch(x8, sc, layers[i % len(layers)][name], M, split, m, out=o)
            floor = int(stamps()[:, 3].max())
            _, tmed = bench.graph_time(torch, fn, args.reps)
            st = stamps()
            sel = (st[:, 0] > floor) & (st[:, :4].min(axis=1) > 0)
            idx = np.nonzero(sel)[0]
            blk = st[sel]
            rel = (blk[:, :4] - blk[:, 0].min()) * (1e3 / khz)  # microseconds
            cu = blk[:, 4]
            _, inv, per_cu = np.unique(cu, return_inverse=True, return_counts=True)
            shared = per_cu[inv]  # blocks of this launch on the block's compute unit
            by_share = {int(k): {"blocks": int((shared == k).sum()),
                                 "t3_p50": round(float(np.median(rel[shared == k, 3])), 3)}
                        for k in np.unique(shared)}
            # round-robin placement: block b on the compute unit of block b mod 256
            cu_of = dict(zip(idx.tolist(), cu.tolist()))
            later = [b for b in idx.tolist() if b >= 256 and b % 256 in cu_of]
            same_cu = (sum(cu_of[b] == cu_of[b % 256] for b in later) / len(later)) if later else None
            span = float(rel[:, 3].max())
            rec = {"launch": name, "M": M, "N": N, "K": K, "split": split, "blocks": int(len(blk)),
                   "us_per_launch": round(tmed, 3), "span_us": round(span, 3),
                   "outside_us": round(tmed - span, 3),
                   "stamps_us": {f"t{i}": {f"p{p}": round(float(np.percentile(rel[:, i], p)), 3) for p in pct}
                                 for i in range(4)},
                   "compute_units": int(len(per_cu)), "t3_by_blocks_per_cu": by_share,
                   "share_cu_with_block_mod_256": same_cu}
            out["launches"].append(rec)
            cols = " | ".join("/".join(f"{rec['stamps_us'][f't{i}'][f'p{p}']:.2f}" for p in pct) for i in range(4))
            print(f"  {name + f' M={M}':<12} {rec['blocks']:>6} {tmed:>9.2f} {span:>6.2f} {tmed - span:>7.2f} | "
                  f"{cols}", flush=True)
            print(f"  {'':<12} on {len(per_cu)} CUs; t3 p50 by blocks per CU: " +
                  ", ".join(f"{k}: {v['t3_p50']:.2f} ({v['blocks']} blocks)" for k, v in by_share.items()) +
                  ("" if same_cu is None else f"; blocks b >= 256 on the CU of block b mod 256: {100 * same_cu:.0f}%"),
                  flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
