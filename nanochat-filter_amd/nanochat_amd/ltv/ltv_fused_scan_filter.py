"""Initialisation helper shared by the combined filters."""

import torch


def init_weights_of_init(init_param, n_head, n_kv_head, init_s):
    """Fill ``init_param`` (H, D) with U(-init_s, init_s), drawing the q rows,
    then the k rows, then the v rows (three separate draws, in that order).

    Same RNG consumption order as the reference
    (``nanochat/ltv/ltv_fused_scan_filter.py:17-39``), so a seeded init gives the
    same values.
    """
    if init_param.shape[0] != n_head + 2 * n_kv_head:
        raise AssertionError("init_param size mismatch")
    q_val = torch.empty_like(init_param[:n_head, :])
    k_val = torch.empty_like(init_param[n_head:n_head + n_kv_head, :])
    v_val = torch.empty_like(init_param[n_head + n_kv_head:n_head + 2 * n_kv_head, :])
    torch.nn.init.uniform_(q_val, -init_s, init_s)
    torch.nn.init.uniform_(k_val, -init_s, init_s)
    torch.nn.init.uniform_(v_val, -init_s, init_s)
    with torch.no_grad():
        init_param.copy_(torch.cat([q_val, k_val, v_val], dim=0))
