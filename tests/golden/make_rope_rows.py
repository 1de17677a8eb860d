"""Write tests/golden/rope.npz: rows of the rope tables at the positions the
golden score fixtures use (every 64-token block start below 32768, and the
queries 32641..32767 of config 5), as the golden generator's build computed
them.

The reference builds its tables with torch on the CPU (reference/layers.py:73-125);
the last bit of a few cos/sin entries depends on the host CPU's math-library
path, so the tests that compare block scores bit for bit against the
fixtures patch these rows in. Run on a build whose full tables reproduce the
digests golden_meta.json records for the reference's own tables (this script
checks that first); the oracle's RotaryEmbedding restates the reference's.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import inputs as gi  # noqa: E402
from oracle.layers import RotaryEmbedding  # noqa: E402


def main():
    meta = json.load(open(os.path.join(HERE, "golden_meta.json")))
    rot = RotaryEmbedding(64, 1e7, [11, 11, 10])
    p = torch.arange(32768)[None]
    cos, sin = rot(p[None].expand(3, -1, -1))
    if gi.digest(cos) != meta["digests"]["rope"]["cos_sha"] or gi.digest(sin) != meta["digests"]["rope"]["sin_sha"]:
        raise SystemExit("this build's rope tables are not the golden generator's: run it where they are")
    positions = np.unique(np.concatenate([np.arange(0, 32768, 64), np.arange(32641, 32768)])).astype(np.int32)
    np.savez_compressed(os.path.join(HERE, "rope.npz"), positions=positions,
                        cos=cos[0, positions].numpy(), sin=sin[0, positions].numpy())
    print("wrote", len(positions), "rows")


if __name__ == "__main__":
    main()
