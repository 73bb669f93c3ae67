"""QXKVSNP1 export/import of the device INT8 cache through the C ABI: a greedy run
interrupted by export -> fresh cache -> import continues with the tokens of the
uninterrupted run, and the exported file holds exactly the device rows."""
import numpy as np
import pytest

import qxg

pytestmark = pytest.mark.gpu


def test_export_import_continues_the_greedy_run(tmp_path):
    p = tmp_path / "m.qxf"
    qxg.generate_model(p, layers=2, vocab=4096, experts=32, seed=44)
    with qxg.Context(0) as c:
        c.load(p)
        c.kv_create(2, 32)
        full, _ = c.generate([17], 10)
        c.kv_create(2, 32)
        first, _ = c.generate([17], 6)          # positions 0..5 cached; first[5] is the next input
        assert list(first) == list(full[:6])
        snap = tmp_path / "kv.bin"
        c.kv_export(snap, 2, 6, 32, int(first[5]), 1)
        k, v, ks, vs, pos, nt = qxg.kvsnap_read(snap, 2, 32, 1)
        assert (pos, nt) == (6, int(first[5]))
        for layer in range(2):
            gk, gv, gks, gvs = c.kv_read(layer, 0, 6)
            assert np.array_equal(gk, k[layer, :6]) and np.array_equal(gv, v[layer, :6])
            assert np.array_equal(gks, ks[layer, :6]) and np.array_equal(gvs, vs[layer, :6])
        c.kv_create(2, 32)                      # a fresh (zeroed) cache
        pos, nt = c.kv_import(snap, 2, 32, 1)
        assert (pos, nt) == (6, int(first[5]))
        rest, _ = c.generate([nt], 4, pos0=pos)
        assert list(rest) == list(full[6:10])
        with pytest.raises(qxg.QxgError, match="header mismatch"):
            c.kv_import(snap, 2, 32, 2)          # wrong seed
