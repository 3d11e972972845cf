"""Writes tests/golden/q4_golden.npz: input blocks and the outputs of the reference's own quantize4
(scripts/export_common.py:64-87), the one function of the path whose tie-breaking no closed form pins.

Run in the development container only (it imports /root/reference/scripts/export_common.py, which never
travels to the GPU box); the .npz it writes is the committed fixture.

    python tests/golden/make_q4_golden.py
"""
import os
import sys

import numpy as np
import torch

REF = "/root/reference/scripts"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4_golden.npz")


def main():
    sys.path.insert(0, REF)
    import export_common  # noqa: E402  (the reference's own quantizers)
    rng = np.random.Generator(np.random.PCG64(1234))
    w = rng.standard_normal((64, 256), dtype=np.float32) * np.float32(0.02)
    w[0, :32] = 0.0                                        # an all-zero block
    w[1, :32] = np.linspace(-1, 1, 32, dtype=np.float32)   # evenly spaced values: near-ties in the search
    w[2, :32] = 0.01                                       # a constant block
    w[3] *= 50                                             # large magnitudes
    w[4, 32:64] = rng.integers(-8, 8, 32).astype(np.float32) * np.float32(0.0123)  # exactly representable codes
    codes4, scales4, deq4 = export_common.quantize4(torch.from_numpy(w))
    np.savez_compressed(OUT, w=w, codes4=codes4, scales4=scales4, deq4=deq4.numpy())
    print(OUT)


if __name__ == "__main__":
    main()
