"""Parity oracle of the GDN layer path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker and the CPU baseline; never by the product
package.  gdn_ref.py restates the reference's algorithm in fp32 torch on the
CPU; recurrence.c is the fp64 token-by-token recurrence that pins it.
"""
import ctypes
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
RECUR_LIB = ORACLE_DIR / "_build" / "liboracle_recur.so"


def build() -> Path:
    """Compile the C oracle with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return RECUR_LIB


def recurrence_f64(q, k, v, g, beta, h0=None, scale=None, l2norm=True):
    """fp64 token recurrence of one sequence via recurrence.c.
    q, k [T, Hk, D]; v [T, Hv, D]; g, beta [T, Hv]; h0 [Hv, D, D] or None.
    Returns (o [T, Hv, D] fp64, final [Hv, D, D] fp64) as torch tensors."""
    import torch

    if not RECUR_LIB.exists():
        build()
    lib = ctypes.CDLL(str(RECUR_LIB))
    T, Hk, D = k.shape
    Hv = v.shape[1]
    qd, kd, vd = (t.double().contiguous() for t in (q, k, v))
    gd, bd = g.double().contiguous(), beta.double().contiguous()
    st = torch.zeros(Hv, D, D, dtype=torch.float64) if h0 is None else h0.double().clone().contiguous()
    out = torch.zeros(T, Hv, D, dtype=torch.float64)
    P = ctypes.c_void_p
    lib.gdn_recurrence_f64.argtypes = [P, P, P, P, P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_double, ctypes.c_int]
    lib.gdn_recurrence_f64(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), gd.data_ptr(), bd.data_ptr(),
                           st.data_ptr(), out.data_ptr(), T, Hk, Hv, D,
                           float(D ** -0.5 if scale is None else scale), int(bool(l2norm)))
    return out, st
