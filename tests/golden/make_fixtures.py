"""Writes tests/golden/c1_fixture.pt from this repository's own CPU oracle.

    python tests/golden/make_fixtures.py

C1 (L2 d128 H4 f512 B2 S64, fp32, lengths U[32,64]): seeded inputs, a
checksum of the seeded weights, and the oracle forward in fp64 and fp32.
The reference ships no golden vectors for this path, so these pin the
oracle against drift; the oracle itself is pinned by tests/test_oracle.py.
Loaded with torch.load(weights_only=True).
"""

import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tiktok-techjam-2026_amd")]

from oracle import model as oracle  # noqa: E402
from tjkernels.workloads import WORKLOADS, make_inputs, make_state_dict  # noqa: E402

PARAM_SEED, INPUT_SEED = 0, 1


def weight_checksum(sd):
    return torch.tensor([[float(v.double().sum()), float((v.double() ** 2).sum())]
                         for _, v in sorted(sd.items())], dtype=torch.float64)


def main():
    w = WORKLOADS["C1"]
    sd = make_state_dict(w, seed=PARAM_SEED)
    x, mask, lengths = make_inputs(w, seed=INPUT_SEED)
    out64 = oracle.forward(sd, x, mask, w.heads, w.causal, torch.float64)
    out32 = oracle.forward(sd, x, mask, w.heads, w.causal, torch.float32)
    blob = {
        "workload": "C1", "param_seed": PARAM_SEED, "input_seed": INPUT_SEED,
        "weight_checksum": weight_checksum(sd),
        "x": x, "mask": mask, "lengths": lengths,
        "out_fp64": out64, "out_fp32": out32,
    }
    path = Path(__file__).with_name("c1_fixture.pt")
    torch.save(blob, path)
    print(f"wrote {path} ({path.stat().st_size} bytes); lengths={lengths.tolist()}")


if __name__ == "__main__":
    main()
