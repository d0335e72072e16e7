"""CPU restatement of EdgeDegreeEmbedding.forward (test oracle only).

Follows src/maloq/helm/nn/embedding.py:82-141 step by step: the RadialMLP
output (one row per degree, the m = 0 coefficients) padded with zeros to the
kept m-major rows (:97-111), einsum with to_m (:114-116), bmm(wigner_inv)
(:120), cast to the dtype of x (:122), then x.index_add_(0, dst, emb /
rescale_factor) (:133-135) or the per-edge embedding (:139-143, no rescale).

The reference runs mmax == lmax; for mmax < lmax the bmm uses the kept
columns ``out_mask`` of wigner_inv (the convention of oracle.message.rotate_out).
For mmax == lmax this is the reference exactly.
"""
from __future__ import annotations

import torch


def edge_degree_embedding(x, x_edge_m0, edge_index, wigner_inv, mapping, out_mask, rescale_factor,
                          node_or_edge="node"):
    """x [N, d, C]; x_edge_m0 [E, (lmax+1) C] (the rad_func output); returns the
    updated copy of x (node) or the embedding [E, d, C] (edge)."""
    m0 = mapping.m_size[0]
    n_all = len(mapping.l_harmonic)
    E = x_edge_m0.shape[0]
    u = x_edge_m0.reshape(E, m0, -1)
    pad = torch.zeros(E, n_all - m0, u.shape[2], dtype=u.dtype)
    emb = torch.cat((u, pad), dim=1)
    emb = torch.einsum("nac,ab->nbc", emb, mapping.to_m.to(emb.dtype))
    emb = torch.bmm(wigner_inv[:, :, out_mask].contiguous().to(emb.dtype), emb)
    emb = emb.to(x.dtype)
    if node_or_edge == "node":
        out = x.clone()
        out.index_add_(0, edge_index[1], emb / rescale_factor)
        return out
    return emb
