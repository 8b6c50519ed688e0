"""Floating-point error bounds for the reassociating (fast) products."""
import numpy as np


def gamma_bound_ok(Y, M, K, ip, ix, vals, X, extra=2):
    """Every output y of a fast (reassociated, fused multiply-add) product is
    within gamma_n * sum_k |w_k x_k| of the exact sum (float64; the products
    of two floats are exact there), n = the row's count + extra: the forward
    error bound that any summation order of n floating-point terms meets
    (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., 3.1;
    `extra` covers the per-row scale applied to an int8 row's sum).  The
    storage-order sum the oracle computes meets the same bound, so the
    two may differ by up to twice it where a row's terms cancel."""
    import scipy.sparse as sparse

    A = sparse.csr_matrix((np.asarray(vals, np.float64), np.asarray(ix), np.asarray(ip)), shape=(M, K))
    Xd = np.asarray(X, np.float64).reshape(K, -1)
    exact = A @ Xd
    absum = abs(A) @ np.abs(Xd)
    n = np.diff(np.asarray(ip)).astype(np.float64)[:, None] + extra
    u = 2.0 ** -24
    gamma = n * u / (1.0 - n * u)
    err = np.abs(np.asarray(Y, np.float64).reshape(M, -1) - exact)
    return bool(np.all(err <= gamma * absum + 1e-30)), float((err / np.maximum(gamma * absum, 1e-300)).max())
