"""Writes mlvc_1920x1088_isa2.json: the CPU oracle's model of the GPU
arithmetic (OraclePlan isa=2: every groups == 1 conv summed as the matrix
core sums it, measured instruction by instruction; everything else the
reference plan) run free-running over the frames of the 1920x1088
MLVC-shaped graph, beside the reference order (isa=0).

Per frame: the SHA-256 of the isa-2 reconstruction (FP16 bytes, NCHW) and
its mean / max |d| relative to the reference-order output RMS. The GPU test
test_mlvc_1920x1088_free_running requires the GPU's frames to hash to these
values, so the free-running difference from the reference order it reports is
the one recorded here, bit for bit.

  python tests/golden/make_mlvc_order_golden.py [--frames 32] [--config mlvc_1920x1088]

(About a minute per frame on 8 CPU threads.)
"""

import argparse
import hashlib
import json
import pathlib
import sys
import tempfile
import time

REPO = pathlib.Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO / "mlvc.cpp_amd" / "python"), str(REPO / "oracle")]

import mlvc_hip  # noqa: E402
import mlvc_oracle  # noqa: E402


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="mlvc_1920x1088")
    ap.add_argument("--frames", type=int, default=32)
    ap.add_argument("--out", type=pathlib.Path, default=None)
    args = ap.parse_args()
    out = args.out or pathlib.Path(__file__).resolve().parent / f"{args.config}_isa2.json"
    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write(args.config, d, 0)
        bindings, _ = mlvc_hip.synth_bindings(args.config)
        model = mlvc_oracle.OraclePlan(d, args.config, bindings, isa=2)
        ref = mlvc_oracle.OraclePlan(d, args.config, bindings, isa=0)
        model.reset_state()
        ref.reset_state()
        frames = []
        for f in range(args.frames):
            t0 = time.time()
            x = mlvc_hip.synth_input(args.config, 0, f, model.in_shapes[0])
            y = model.run([x])[0]
            st = mlvc_oracle.parity_stats(y, ref.run([x])[0])
            frames.append({"frame": f, "sha256": hashlib.sha256(y.tobytes()).hexdigest(),
                           "mean_rel_vs_reference_order": st["mean_rel"],
                           "max_rel_vs_reference_order": st["max_rel"]})
            print(f"frame {f}: mean {st['mean_rel']:.4e} max {st['max_rel']:.4e} ({time.time() - t0:.0f} s)", flush=True)
        out.write_text(json.dumps({"config": args.config, "seed": 0, "input": "mlvc_hip.synth_input(config, 0, frame)",
                                   "threads": model.threads, "frames": frames}, indent=1) + "\n")
    print(f"wrote {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
