"""Demote selection on the device (akv_select_demote) vs the oracle's restatement of
AKVLayer._select_demote_indices (akv/drop_in.py:392-413): exact index lists."""
import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev
from oracle import selection as osel

pytestmark = pytest.mark.gpu


def _check(imp, n, hot_len, budget):
    from akv.drop_in import select_demote_indices
    got = select_demote_indices(to_dev(imp), n, hot_len, budget).cpu().numpy()
    imp2 = np.atleast_2d(imp)
    ref = np.stack([osel.select_demote_indices(r, n, hot_len, budget) for r in imp2])
    assert got.reshape(ref.shape).tolist() == ref.tolist()


@pytest.mark.parametrize("rows,hot_len,n,budget", [(3, 1000, 900, 64), (1, 4096, 1, 128), (2, 257, 256, 8),
                                                   (5, 33, 0, 64)])
def test_select_random(rows, hot_len, n, budget):
    announce(f"select rows={rows} len={hot_len} n={n}")
    imp = np.random.default_rng(hot_len + n).random((rows, hot_len)).astype(np.float32)
    _check(imp, n, hot_len, budget)


def test_select_ties_nan_signed_zero():
    """Equal scores take the lower index; NaN sorts above +inf; -0 equals +0."""
    announce("select ties / NaN / signed zero")
    rng = np.random.default_rng(3)
    imp = rng.integers(0, 6, size=(4, 300)).astype(np.float32)
    imp[0, 10:20] = np.nan
    imp[1, ::7] = -0.0
    imp[2, :] = 1.0
    _check(imp, 250, 300, 64)
    _check(imp, 300, 300, 64)  # every position, protected ones last


def test_select_single_row_and_fifo():
    from akv.drop_in import select_demote_indices
    announce("select 1-D scores and the FIFO rule")
    imp = np.random.default_rng(4).random(500).astype(np.float32)
    _check(imp, 400, 500, 64)
    assert select_demote_indices(to_dev(imp), 10, 499, 64).cpu().tolist() == list(range(10))


def test_select_demote_64k_shape():
    announce("select 16 x 65536, 64512 demoted")
    imp = np.random.default_rng(5).random((16, 65536)).astype(np.float32)
    _check(imp, 64512, 65536, 64)
