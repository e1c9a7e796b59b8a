"""Writes the golden fixtures of this directory.

philox4x32_10_kat.json: the Philox4x32-10 known-answer vectors published
  with Random123 (Salmon, Moraes, Dror, Shaw, SC'11; the kat_vectors file of
  the Random123 distribution): counter words, key words, output words.
e4m3fn_codes.json: the value of every OCP float8_e4m3fn code as torch
  decodes it (torch.float8_e4m3fn viewed from the byte, widened to float32),
  as float32 bit patterns.

Run from the repository root:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

PHILOX_KAT = [
    {"ctr": [0x00000000, 0x00000000, 0x00000000, 0x00000000], "key": [0x00000000, 0x00000000],
     "out": [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]},
    {"ctr": [0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF], "key": [0xFFFFFFFF, 0xFFFFFFFF],
     "out": [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]},
    {"ctr": [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], "key": [0xA4093822, 0x299F31D0],
     "out": [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]},
]


def main() -> None:
    with open(os.path.join(HERE, "philox4x32_10_kat.json"), "w") as fh:
        json.dump({"source": "Random123 kat_vectors, philox4x32_10", "vectors": PHILOX_KAT}, fh, indent=1)
        fh.write("\n")

    import numpy as np
    import torch

    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    with open(os.path.join(HERE, "e4m3fn_codes.json"), "w") as fh:
        json.dump({"source": f"torch {torch.__version__} float8_e4m3fn -> float32",
                   "f32_bits": [f"{int(b):08x}" for b in vals.view(np.uint32)]}, fh, indent=0)
        fh.write("\n")


if __name__ == "__main__":
    main()
