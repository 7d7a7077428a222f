"""Writes tests/golden/c5_100_steps.json: the CPU oracle's run of config C5 for 100 steps.

C5 is the strict F32 MLP 1024 -> 4096 -> 4096 -> 1024 with ReLU hidden activations, batch
4096, MSE against a uniform[-1, 1) target, reverse mode, and strict SGD at lr 1e-3, with
the weights fed back after every step. Inputs come from the seeded generator in
fusion-pcu_amd/synthetic.py (X seed 51, Y seed 52, W1..W3 seeds 53..55, Xavier-uniform),
the same arrays the GPU test builds.

Each step is evaluated by the oracle's graph restatement (oracle/graph.py: the
reference's builder, backward_mse and plan order) with the fast oracle ops, whose
equality with the faithful integer law is tested on the CPU. The fixture keeps, per step,
the loss bit pattern and a SHA-256 of each updated weight tensor's bytes (little-endian
binary32), so a GPU run can be compared bit for bit at every step without shipping
100 x 84 MiB of weights. About 10 minutes on 8 host cores.

Run: python tests/golden/make_c5_fixture.py
"""
import hashlib
import importlib.util
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from oracle import graph as og  # noqa: E402

DIMS, BATCH, LR, STEPS = (1024, 4096, 4096, 1024), 4096, 1e-3, 100
SEEDS = {"x": 51, "y": 52, "w": (53, 54, 55)}


def _synthetic():
    path = os.path.join(ROOT, "fusion-pcu_amd", "synthetic.py")
    spec = importlib.util.spec_from_file_location("pcu_synthetic", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f4").tobytes()).hexdigest()


def main() -> None:
    syn = _synthetic()
    x = syn.uniform(SEEDS["x"], (BATCH, DIMS[0]), np.float32)
    y = syn.uniform(SEEDS["y"], (BATCH, DIMS[3]), np.float32)
    ws = [syn.xavier_uniform(SEEDS["w"][i], DIMS[i], DIMS[i + 1], np.float32) for i in range(3)]
    g, ids = og.mlp_graph(DIMS, BATCH, np.float32, LR)
    steps = []
    t0 = time.time()
    for it in range(STEPS):
        vals, fault = g.evaluate({ids["x"]: x, ids["w1"]: ws[0], ids["w2"]: ws[1],
                                  ids["w3"]: ws[2], ids["y"]: y}, ids["outputs"])
        if fault is not None:
            raise SystemExit(f"step {it}: oracle fault {fault}")
        ws = [vals[o] for o in ids["outputs"][:3]]
        loss = vals[ids["outputs"][3]]
        steps.append({"loss": "0x%08x" % int(np.asarray(loss, np.float32).view(np.uint32)),
                      "w_sha256": [digest(w) for w in ws]})
        print(f"step {it} loss {float(loss):.9g} ({time.time() - t0:.0f} s)", flush=True)
    out = {
        "config": "C5 strict F32 MLP 1024-4096-4096-1024, batch 4096, lr 1e-3",
        "seeds": SEEDS,
        "generator": "fusion-pcu_amd/synthetic.py (SplitMix64 uniform / Xavier-uniform)",
        "checker": "oracle/graph.py mlp_graph evaluated with the fast oracle ops",
        "digest": "SHA-256 of each updated weight's little-endian binary32 bytes",
        "steps": steps,
    }
    with open(os.path.join(HERE, "c5_100_steps.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
