"""Synthetic batch generator: structure and termination (CPU)."""
import time

import numpy as np

from tatara_amd.synthetic import HALFKA_HM_MERGED, HALFKP, small_spec, structured_batch


def test_rows_are_distinct_and_king_blocked():
    for spec, n in ((small_spec(6, 64, 40), 2048), (small_spec(10, 64, 40), 512), (HALFKA_HM_MERGED, 4096), (HALFKP, 4096)):
        t0 = time.time()
        b, bucket = structured_batch(n, spec, num_buckets=8, seed=3)
        assert time.time() - t0 < 10
        for idx in (b.stm_indices, b.nstm_indices):
            assert idx.shape == (n, spec["max_active"])
            valid = idx >= 0
            assert (idx[valid] < spec["ft_in"]).all()
            s = np.sort(idx, axis=1)
            assert not ((s[:, 1:] == s[:, :-1]) & (s[:, 1:] >= 0)).any()
            kb = np.where(valid, idx // spec["piece_inputs"], -1)
            first = kb[:, :1]
            assert ((kb == first) | ~valid).all()
        assert ((bucket >= 0) & (bucket < 8)).all()
        assert np.abs(b.score).max() <= 3000 and set(np.unique(b.wdl)) <= {0.0, 0.5, 1.0}
