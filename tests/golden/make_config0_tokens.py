"""Writes tests/golden/config0_tokens.txt: the configs[0] greedy tokens of the
CPU oracle's decoder (weights N(0, 0.02) from PCG64 seed 0 in the parameter
order of include/rustral_model.h, prompt of 32 ids from numpy's
default_rng(0).integers(0, 1000), 64 new tokens), as plain text so a test
without a JSON parser (the Rust crate's) can read it.

Run from the repo root: python tests/golden/make_config0_tokens.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def tokens():
    import oracle
    from rustral_amd import model
    cfg = model.config()
    params = model.init_params(cfg, seed=0, std=0.02)
    prompt = np.random.default_rng(0).integers(0, 1000, 32).astype(np.int32)
    want = oracle.decoder_generate(oracle.decoder_config(), params, prompt, 64)
    return prompt, want


def main():
    prompt, want = tokens()
    with open(os.path.join(HERE, "config0_tokens.txt"), "w") as f:
        f.write("# configs[0]: seed 0 weights N(0, 0.02), prompt default_rng(0), 64 greedy tokens\n")
        f.write("prompt " + " ".join(str(int(t)) for t in prompt) + "\n")
        f.write("tokens " + " ".join(str(int(t)) for t in want) + "\n")


if __name__ == "__main__":
    main()
