"""Series primitives of the oracle (test infrastructure only; see oracle/__init__.py).

Every function takes and returns lists of K+1 ordinary CPU tensors
(coefficients of ``sum_k X_k t^k``) and follows the reference's plain-range
rules operation for operation.
"""

import torch


def cauchy(left, right, matmul=False):
    """Truncated product: C_k = sum_{i=0..k} L_i (*|@) R_{k-i}, accumulated in increasing i.

    /root/reference/src/polytensors/_plain.py:118-128 (plain_polynomial_product);
    matrix pairs promote both operands first (_plain.py:77-80).
    """
    out = []
    for k in range(len(left)):
        total = None
        for i in range(k + 1):
            a, b = left[i], right[k - i]
            if matmul:
                dtype = torch.promote_types(a.dtype, b.dtype)
                term = torch.matmul(a.to(dtype), b.to(dtype))
            else:
                term = a * b
            total = term if total is None else total + term
        out.append(total)
    return out


def quotient(A, B):
    """Elementwise series quotient: Q_k = (A_k - sum_{i=1..k} B_i Q_{k-i}) / B_0.

    /root/reference/src/polytensors/_range_ops.py:86-93 (quotient).
    """
    out = []
    for k in range(len(A)):
        remainder = A[k]
        for i in range(1, k + 1):
            remainder = remainder - B[i] * out[k - i]
        out.append(remainder / B[0])
    return out


def exp_series(X):
    """exp along a series: Y_0 = exp(X_0), Y_k = sum_{i=1..k} (i/k) X_i Y_{k-i}.

    /root/reference/src/polytensors/_plain.py:153-159 (plain_exp).
    """
    Y = [torch.exp(X[0])]
    for k in range(1, len(X)):
        acc = None
        for i in range(1, k + 1):
            term = (i / k) * X[i] * Y[k - i]
            acc = term if acc is None else acc + term
        Y.append(acc)
    return Y


def log_series(X):
    """log along a series: Y_0 = log X_0, with n_k = X_k / X_0,
    Y_k = n_k - sum_{i=1..k-1} (i/k) Y_i n_{k-i}.

    /root/reference/src/polytensors/_plain.py:162-171 (plain_log).
    """
    Y = [torch.log(X[0])]
    n = [None] + [x / X[0] for x in X[1:]]
    for k in range(1, len(X)):
        acc = n[k]
        for i in range(1, k):
            acc = acc - (i / k) * Y[i] * n[k - i]
        Y.append(acc)
    return Y


def rsqrt_series(X):
    """rsqrt along a series: Y_0 = rsqrt(X_0), with n_k = X_k / X_0,
    Y_k = -sum_{i=1..k} ((2k-i)/(2k)) n_i Y_{k-i}.

    /root/reference/src/polytensors/_series.py:83-96 (SeriesOps.poly_rsqrt).
    """
    Y = [torch.rsqrt(X[0])]
    n = [None] + [x / X[0] for x in X[1:]]
    for k in range(1, len(X)):
        acc = ((2 * k - 1) / (2 * k)) * n[1] * Y[k - 1]
        for i in range(2, k + 1):
            acc = acc + ((2 * k - i) / (2 * k)) * n[i] * Y[k - i]
        Y.append(-acc)
    return Y


def softmax_family(X, dim):
    """(softmax, log_softmax, logsumexp-keepdim) series along ``dim``.

    /root/reference/src/polytensors/_plain.py:262-273 (plain_softmax_family):
    lse_0 = logsumexp(X_0); E = exp series of [X_0 - lse_0, X_1..X_K];
    Z_k = sum(E_k); log_z = log series of Z; log_softmax_k = X_k - log_z_k
    (k >= 1, order 0 native); softmax = exp series of log_softmax with order 0
    native; lse = [lse_0, log_z_1..log_z_K].
    """
    lse0 = torch.logsumexp(X[0], dim=dim, keepdim=True)
    centered = [X[0] - lse0] + list(X[1:])
    E = exp_series(centered)
    Z = [e.sum(dim=dim, keepdim=True) for e in E]
    log_z = log_series(Z)
    log_softmax = [torch.log_softmax(X[0], dim=dim)] + [c - l for c, l in zip(centered[1:], log_z[1:])]
    softmax = exp_series(log_softmax)
    softmax[0] = torch.softmax(X[0], dim=dim)
    lse = [lse0] + list(log_z[1:])
    return softmax, log_softmax, lse
