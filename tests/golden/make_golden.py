"""Write the golden index fixtures of this directory from the oracle.

    python tests/golden/make_golden.py

Fixtures (inputs and expected outputs of the index construction, kept so that
any later change to the sampler or the tile map shows up as a test failure):
  bell_col_idx_cfg2.npy   sample_col_idx(seed=0, 40 block-rows, 160 block-cols, width 40)
  bell_col_idx_cfg4.npy   sample_col_idx(seed=4, 10 block-rows, 40 block-cols, width 20)
  wattn_tiles_cfg3.npy    64x64 tile kinds of the band mask, S=4096, w=512, Np=16, causal
  wattn_worklist_cfg3.npz kernel work list (q_block 128, sub_rows 32) of the same mask
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import block_ell as ob  # noqa: E402
from oracle import masks as om  # noqa: E402


def main() -> None:
    np.save(HERE / "bell_col_idx_cfg2.npy", ob.sample_col_idx(0, 40, 160, 40))
    np.save(HERE / "bell_col_idx_cfg4.npy", ob.sample_col_idx(4, 10, 40, 20))
    m = om.band_mask(4096, 512, 16)
    np.save(HERE / "wattn_tiles_cfg3.npy", om.tile_kinds(m, 64, 64))
    rp, ent = om.schedule(m, 128, 32, 64)
    np.savez(HERE / "wattn_worklist_cfg3.npz", row_ptr=rp, entries=ent)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
