"""Write tests/golden/config1_b0h0.npz: config 1's golden O, LSE, dQ, dK, dV.

Config 1 is causal attention, B=2, H=4, L=256, d=64 in fp32
with Q/K/V/dO ~ N(0, 1) from seed 0 (kerneldev_amd.synth.config_inputs).
The fixture keeps head (b=0, h=0) of the fp64 dense oracle
(oracle/attention.py) plus a SHA-256 of the seeded inputs, so a test can
check that it regenerates the very same inputs before comparing.  The
reference ships no golden vectors of its own (it has no tests), so these are
the oracle's, recorded once so later changes to the oracle or the inputs are
caught.

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from kerneldev_amd.synth import config_inputs  # noqa: E402
from oracle import attention as ref  # noqa: E402
from oracle.mask import dense_mask  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1_b0h0.npz")


def input_digest(inp) -> str:
    h = hashlib.sha256()
    for name in ("q", "k", "v", "do"):
        h.update(inp[name].contiguous().numpy().tobytes())
    return h.hexdigest()


def golden():
    inp = config_inputs(1, seed=0)
    q, k, v, do = (inp[x][0:1, 0:1] for x in ("q", "k", "v", "do"))
    T, D = q.shape[2], q.shape[3]
    mask = torch.from_numpy(dense_mask(T, B=1, causal=True))
    o, lse = ref.forward(q, k, v, mask, D ** -0.5)
    dq, dk, dv, _ = ref.backward(q, k, v, o, do, mask, D ** -0.5)
    return inp, {"o": o[0, 0].numpy(), "lse": lse[0, 0].numpy(), "dq": dq[0, 0].numpy(),
                 "dk": dk[0, 0].numpy(), "dv": dv[0, 0].numpy()}


if __name__ == "__main__":
    inp, g = golden()
    np.savez_compressed(OUT, digest=np.array(input_digest(inp)), **g)
    print("wrote", OUT)
