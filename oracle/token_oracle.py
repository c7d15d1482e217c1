"""CPU float64 restatement of the token-cached EWS scan (the reference's ews/core/token_scan.py).

TEST INFRASTRUCTURE ONLY. Nothing in the product imports, links or runs this file; ``tests/`` use it as the
checker of the HIP token-cache kernels. Torch float64, gradients from autograd; every function cites the reference
file:line it restates.
"""

from __future__ import annotations

import torch

from oracle import ews_oracle as O

DT = torch.float64


def build_token_cache(vocab_dx, vocab_dtheta, A, M, N, expm_method="exact", chen_expm_method=None,
                      leaf="van_loan", series_q=None):
    """ews/core/token_scan.py:44-88: the packed local signature of each token's segment (displacement vocab_dx[g],
    clock increment vocab_dtheta[g]) with the layer's leaf, and its flow exp(-dtheta_g A) with chen_expm."""
    chen = expm_method if chen_expm_method is None else chen_expm_method
    if leaf == "series":
        local = O.series_local_terms(vocab_dx, vocab_dtheta, A, N, int(series_q))
    elif leaf == "van_loan":
        local = O.van_loan_local_terms(vocab_dx, vocab_dtheta, A, N, M, expm_method, "displacement")
    else:
        raise ValueError(leaf)
    return O.pack(local), O.flows(vocab_dtheta, A, chen)


def token_cached_prefix_scan(token_ids, mask, P_cache, D_cache, dim, trunc):
    """ews/core/token_scan.py:91-118 for one sample: D_t = D_cache[g_t] (identity on a padded step),
    P_t = P_cache[g_t] (the unit signature on a padded step), S_t = mult(apply_M(S_{t-1}, D_t), P_t) from the unit.
    Returns the packed prefix (L, sum_k d^k)."""
    L = token_ids.shape[0]
    on = torch.ones(L, dtype=torch.bool) if mask is None else mask.to(torch.bool)
    P = torch.where(on[:, None], P_cache[token_ids], torch.zeros_like(P_cache[token_ids]))
    eye = torch.eye(dim, dtype=D_cache.dtype).expand(L, dim, dim)
    D = torch.where(on[:, None, None], D_cache[token_ids], eye)
    return O.chen_scan_prefix(O.unpack(P, dim, trunc), D)


def token_cached_prefix_scan_depth1(token_ids, mask, P_cache, D_cache):
    """ews/core/token_scan.py:91-118 at trunc 1, batched: token_ids (B, L), mask (B, L) or None -> (B, L, d).
    At depth 1 mult(apply_M(S, D), P) is D S + P, so the scan is S_t = D_{g_t} S_{t-1} + P_{g_t} from zero, a padded
    step keeping the state. Pinned to token_cached_prefix_scan (the packed Chen loop) in tests/test_oracle_token.py."""
    B, L = token_ids.shape
    on = torch.ones(B, L, dtype=torch.bool) if mask is None else mask.to(torch.bool).expand(B, L)
    S = torch.zeros(B, P_cache.shape[1], dtype=P_cache.dtype)
    rows = []
    for t in range(L):
        g = token_ids[:, t]
        nxt = torch.bmm(D_cache[g], S[:, :, None])[:, :, 0] + P_cache[g]
        S = torch.where(on[:, t, None], nxt, S)
        rows.append(S)
    return torch.stack(rows, 1)
