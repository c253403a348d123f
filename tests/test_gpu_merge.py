"""The log-sum-exp merges of split partials against the oracle's merge: the one-set merge
(pk_merge_partials: up to 8, up to 128 and more partials per row, and head_dims below 16,
take different kernels) and the merge over sets whose rows are numbered differently
(pk_merge_partial_sets, what the input-chunk attention uses)."""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao

pytestmark = pytest.mark.gpu


def _partials(g, rows, n, hd, masked=0.0):
    """Random (m, l, acc) [rows, n(, hd)] as a split decode writes them; a fraction of
    the partials are empty (m = -inf, l = 0, acc = 0) but never all of one row."""
    m = torch.randn(rows, n, generator=g, dtype=torch.float64) * 4
    l = torch.rand(rows, n, generator=g, dtype=torch.float64) * 30 + 0.5
    acc = torch.randn(rows, n, hd, generator=g, dtype=torch.float64) * l[..., None]
    if masked:
        empty = torch.rand(rows, n, generator=g) < masked
        empty[:, 0] = False
        m[empty] = -np.inf
        l[empty] = 0
        acc[empty] = 0
    return m, l, acc


def _oracle(sets):
    """Per output row, the list of (m, l, acc) columns of every set."""
    parts = []
    for m, l, acc in sets:
        parts += [(m[:, c], l[:, c], acc[:, c]) for c in range(m.shape[1])]
    return ao.merge_partials(parts, out_dtype=None)


@pytest.mark.parametrize("rows,n,hd", [(3000, 1, 128), (3000, 2, 128), (700, 5, 64),
                                       (448, 8, 128), (448, 10, 128), (448, 16, 128),
                                       (280, 17, 128), (28, 35, 128), (28, 64, 64),
                                       (28, 65, 128), (14, 128, 64), (28, 150, 128),
                                       (20, 40, 8), (14, 5, 64), (28, 1, 128)])
def test_merge_partials_matches_the_oracle(gpu, rows, n, hd):
    from phasekv_amd import decode as dec
    print(f"case rows={rows} n={n} hd={hd}", flush=True)
    g = torch.Generator().manual_seed(rows + n + hd)
    m, l, acc = _partials(g, rows, n, hd, masked=0.2 if n > 1 else 0.0)
    want = _oracle([(m.numpy(), l.numpy(), acc.numpy())])
    dm, dl, dacc = (t.float().to(gpu) for t in (m, l, acc))
    out = dec.merge_partials(dm, dl, dacc, normalize=True)
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=2e-3, rtol=2e-3)
    om, ol, oacc = dec.merge_partials(dm, dl, dacc, normalize=False)
    np.testing.assert_allclose(om.cpu().numpy(), m.max(dim=1).values.numpy(), rtol=1e-6)
    got = oacc.cpu().double().numpy() / ol.cpu().double().numpy()[:, None]
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("T,hq,hd,na,nb", [(256, 28, 128, 3, 1), (37, 28, 128, 4, 11),
                                           (5, 8, 64, 1, 2), (1, 8, 64, 20, 1)])
def test_merge_partial_sets_reads_each_set_in_its_own_row_order(gpu, T, hq, hd, na, nb):
    """Set a holds rows (head, token), set b rows (token, head), as the input-chunk
    attention's two launches write them; the output is [token, head]."""
    from phasekv_amd import decode as dec
    print(f"case T={T} hq={hq} hd={hd} na={na} nb={nb}", flush=True)
    g = torch.Generator().manual_seed(T * hq + na + nb)
    a = _partials(g, hq * T, na, hd, masked=0.25)
    b = _partials(g, T * hq, nb, hd, masked=0.25)
    # the oracle merges row (t, h): row h * T + t of a, row t * hq + h of b
    a_th = [x.view(hq, T, *x.shape[1:]).transpose(0, 1).reshape(T * hq, *x.shape[1:]).numpy()
            for x in a]
    want = _oracle([a_th, [x.numpy() for x in b]]).reshape(T, hq, hd)
    da = tuple(x.float().to(gpu).contiguous() for x in a)
    db = tuple(x.float().to(gpu).contiguous() for x in b)
    out = dec.merge_partial_sets([(da, 1, T), (db, hq, 1)], T, hq)
    assert out.shape == (T, hq, hd) and out.dtype == torch.float16
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=2e-3, rtol=2e-3)
    om, ol, oacc = dec.merge_partial_sets([(da, 1, T), (db, hq, 1)], T, hq, normalize=False)
    got = (oacc.cpu().double() / ol.cpu().double()[:, None]).numpy().reshape(T, hq, hd)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
    # a single set with the identity order is the one-set merge
    one = dec.merge_partial_sets([(db, hq, 1)], T, hq)
    ref = dec.merge_partials(*db, normalize=True).view(T, hq, hd)
    np.testing.assert_allclose(one.float().cpu().numpy(), ref.float().cpu().numpy(),
                               atol=1e-3, rtol=1e-3)


def test_merge_partial_sets_rejects_strides_past_the_rows(gpu):
    from phasekv_amd import decode as dec
    g = torch.Generator().manual_seed(5)
    a = tuple(x.float().to(gpu) for x in _partials(g, 40, 2, 64))
    with pytest.raises(ValueError, match="past its rows"):
        dec.merge_partial_sets([(a, 1, 6)], 5, 8)        # last row 4 + 7 * 6 = 46 of 40
    dec.merge_partial_sets([(a, 8, 1)], 5, 8)
    with pytest.raises(ValueError, match="partial sets"):
        dec.merge_partial_sets([(a, 8, 1)] * 5, 5, 8)
