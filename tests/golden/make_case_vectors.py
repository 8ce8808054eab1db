"""Write tests/golden/organizer_cases_v1.npz from the organizer's case generator.

Usage (in the build container only, where the reference checkout exists):

    python tests/golden/make_case_vectors.py [/root/reference]

The accuracy harness draws every trial's input and key-padding mask with the
organizer's ``generate_random_case``
(benchmarks/torch_transformer_benchmark.py:234-272).  The oracle
(oracle/model.py) and the product (transformer_opt/submission.py) restate
that generator from its source text; no library routine or closed form pins
its draw order (randn, then randint over ``[round(S*(1-ratio)), S]``), the
bounds of ``randint`` or Python's round-half-to-even.  This script imports
the organizer's function itself, on the CPU, and stores what it returns for a
grid of seeds, padding ratios, input scales and dtypes, so
tests/test_oracle.py can compare both restatements with it bit for bit.

Only this function of the reference is imported; nothing of the reference is
copied into the fixture except the generator's outputs.  The GPU box never
runs this script (the reference checkout does not exist there).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "organizer_cases_v1.npz"

RATIOS = (0.0, 0.3, 0.5, 0.9, 1.0)
SEEDS = (0, 7, 1234)


def cases():
    """(batch, seq_len, d_model, ratio, seed, scale, dtype) of every stored case.

    One ordinary shape over every dtype and two input scales; one with many
    sequences per ``randint`` draw; two where ``round(S * (1 - ratio))`` lands
    on a .5 tie (S=5 and S=7 at ratio 0.5).
    """
    for ratio in RATIOS:
        for seed in SEEDS:
            for dtype in (torch.float32, torch.bfloat16, torch.float16):
                for scale in (1.0, 2.5):
                    yield 3, 16, 4, ratio, seed, scale, dtype
            yield 32, 24, 1, ratio, seed, 1.0, torch.float32
            yield 4, 5, 6, ratio, seed, 1.0, torch.float32
            yield 2, 7, 3, ratio, seed, 1.5, torch.bfloat16


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    from benchmarks.torch_transformer_benchmark import TransformerConfig, generate_random_case

    arrays = {}
    index = []
    for batch, seq_len, d_model, ratio, seed, scale, dtype in cases():
        config = TransformerConfig(batch, seq_len, d_model, 1, 1, 1, False)
        x, mask = generate_random_case(config, torch.device("cpu"), dtype, seed, ratio, scale)
        key = f"c{len(index)}"
        arrays[f"{key}_x"] = x.float().numpy()
        arrays[f"{key}_mask"] = mask.numpy()
        index.append((batch, seq_len, d_model, ratio, seed, scale,
                      str(dtype).replace("torch.", "")))
    arrays["index"] = np.array([repr(row) for row in index])
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(index)} cases to {OUT}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
