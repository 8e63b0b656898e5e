"""Acceptance criteria for GPU GEMM results against the CPU oracle.

Three checks, all against oracle outputs on the same inputs:

1. normalised error vs the exact (fp64) result, judged against the magnitude
   the accumulation went through, sum_k |a_k b_k| (the analogue of the
   reference's c_peak criterion, rtl_verification/check.py:158-215).  The
   GPU kernels round at most once per 16-element block plus a short tree
   (GEMV: K/64 sequential fmas per lane + 6 reduction levels; MFMA: one fp32
   accumulate per 32-element instruction), so the bound is
   (K/16 + 16) * 2^-24.  A dropped or doubled term moves the error by about
   1/K of the magnitude sum, far above the bound.
2. the same against the reference's portable scalar GEMM (kernels_scalar.c),
   which itself rounds K times: bound (K + K/16 + 16) * 2^-24.
3. the required strict per-element relative error of 1e-3 against the
   scalar reference, on every element whose |ref| >= 1e-3 * sum|ab|; the
   others (near-total cancellation) are counted and reported, and covered by
   checks 1 and 2.
"""
import numpy as np

import oracle

U = 2.0 ** -24
REL_TOL = 1e-3          # the required per-element relative error bound
NEAR_ZERO = 1e-3        # |ref| < NEAR_ZERO * sum|ab| is excluded from the strict check


def pick_rows(M, limit):
    if M <= limit:
        return np.arange(M)
    rows = np.unique(np.concatenate([np.arange(4), np.linspace(0, M - 1, limit - 8).astype(int),
                                     np.arange(M - 4, M)]))
    return rows


def compare(c_gpu, a, b, M, K, N, rows=None, cols=None, gated_up=None):
    """Check c_gpu [M,N] against the oracle on a subset of rows/cols.

    a: fp32 [M*K] (any values; the oracle reference rounds it to bf16 first,
    as the GPU does); b: bf16 bits [N*K].  Returns a dict of the measured
    error figures; raises AssertionError on failure."""
    a = np.asarray(a, np.float32).reshape(M, K)
    b = np.asarray(b, np.uint16).reshape(N, K)
    rows = np.arange(M) if rows is None else np.asarray(rows)
    cols = np.arange(N) if cols is None else np.asarray(cols)
    ar = oracle.round_bf16(np.ascontiguousarray(a[rows]))
    bc = np.ascontiguousarray(b[cols])
    m, n = len(rows), len(cols)
    exact, absum = oracle.gemm_exact(ar, bc, m, K, n)
    ref = oracle.gemm_scalar(ar, bc, m, K, n)
    got = np.asarray(c_gpu, np.float32).reshape(M, N)[np.ix_(rows, cols)].astype(np.float64)
    denom = np.maximum(absum, 1e-30)
    nerr_exact = float(np.max(np.abs(got - exact) / denom)) if got.size else 0.0
    nerr_ref = float(np.max(np.abs(got - ref) / denom)) if got.size else 0.0
    mask = np.abs(ref) >= NEAR_ZERO * absum
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    max_rel = float(np.max(rel[mask])) if mask.any() else 0.0
    info = {"nerr_exact": nerr_exact, "nerr_ref": nerr_ref, "max_rel": max_rel,
            "excluded": int((~mask).sum()), "checked": int(mask.sum()),
            "bitexact_frac": float(np.mean(got.astype(np.float32).view(np.uint32) ==
                                           ref.view(np.uint32))) if got.size else 1.0}
    assert np.all(np.isfinite(got)), "non-finite GPU output"
    assert nerr_exact <= (K / 16 + 16) * U, info
    assert nerr_ref <= (K + K / 16 + 16) * U, info
    assert max_rel <= REL_TOL, info
    return info


def compare_gated(h_gpu, x, wg, wu, M, K, N, rows=None, cols=None):
    """h = silu(x.wg^T) * (x.wu^T): compare against the oracle's scalar
    gate/up GEMMs followed by the reference silu_mul.  The error of h is
    bounded by propagating the GEMM bounds through silu(g)*u:
    |dh| <= |silu'(g)| |u| dg + |silu(g)| du  (silu' <= 1.1), plus a few ulps
    of expf and the divide."""
    x = np.asarray(x, np.float32).reshape(M, K)
    rows = np.arange(M) if rows is None else np.asarray(rows)
    cols = np.arange(N) if cols is None else np.asarray(cols)
    xr = oracle.round_bf16(np.ascontiguousarray(x[rows]))
    g_rows = np.ascontiguousarray(np.asarray(wg, np.uint16).reshape(N, K)[cols])
    u_rows = np.ascontiguousarray(np.asarray(wu, np.uint16).reshape(N, K)[cols])
    m, n = len(rows), len(cols)
    g, ga = oracle.gemm_exact(xr, g_rows, m, K, n)
    u, ua = oracle.gemm_exact(xr, u_rows, m, K, n)
    gs = oracle.gemm_scalar(xr, g_rows, m, K, n)
    us = oracle.gemm_scalar(xr, u_rows, m, K, n)
    ref = oracle.silu_mul(gs.ravel(), us.ravel()).reshape(m, n).astype(np.float64)
    got = np.asarray(h_gpu, np.float32).reshape(M, N)[np.ix_(rows, cols)].astype(np.float64)
    bound_g = (K + K / 16 + 16) * U * ga
    bound_u = (K + K / 16 + 16) * U * ua
    silu = g / (1 + np.exp(-g))
    tol = 1.1 * np.abs(u) * bound_g + np.abs(silu) * bound_u + 8 * U * np.abs(ref) + 1e-30
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got)), "non-finite GPU output"
    worst = float(np.max(err / tol))
    mask = np.abs(ref) >= NEAR_ZERO * (np.abs(silu) * ua + np.abs(u) * ga + 1e-30)
    rel = err / np.maximum(np.abs(ref), 1e-30)
    max_rel = float(np.max(rel[mask])) if mask.any() else 0.0
    info = {"worst_over_bound": worst, "max_rel": max_rel, "excluded": int((~mask).sum())}
    assert worst <= 1.0, info
    assert max_rel <= REL_TOL, info
    return info
