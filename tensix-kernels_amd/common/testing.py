"""The test bars of the reference (common/testing.py:16-41 of XylolabsInc/tensix-kernels), for torch tensors.

check: relative Frobenius error below rel and PCC above pcc, every value finite. same: bit for bit. raises: the
exception type. Each prints one `ok` / `FAIL` line in the reference's format.
"""

import torch


def check(name, y, r, rel=0.01, pcc=0.9999):
    """y against the reference r: relative Frobenius error below rel and PCC above pcc, every value finite. Both are
    computed in float64: a float32 correlation over millions of values carries summation error of the order of the
    bar itself (it moves with the BLAS blocking and thread count)."""
    y, r = y.detach().cpu().double(), r.detach().cpu().double()
    e = ((y - r).norm() / r.norm()).item()
    p = torch.corrcoef(torch.stack([y.flatten(), r.flatten()]))[0, 1].item()
    ok = bool(torch.isfinite(y).all()) and e < rel and p > pcc
    print(f"{'ok  ' if ok else 'FAIL'} {name}: rel {100 * e:.4f} % pcc {p:.6f}", flush=True)
    assert ok, (name, e, p)
    return e


def same(name, a, b):
    """a and b bit for bit."""
    a, b = a.detach().cpu(), b.detach().cpu()
    ok = a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b)
    print(f"{'ok  ' if ok else 'FAIL'} {name}: bit for bit {'equal' if ok else 'DIFFERENT'}", flush=True)
    assert ok, name


def raises(name, exc, fn):
    """fn() raises exc."""
    try:
        fn()
    except exc as e:
        print(f"ok   {name}: {type(e).__name__}", flush=True)
        return
    print(f"FAIL {name}: no {exc.__name__}", flush=True)
    raise AssertionError(name)
