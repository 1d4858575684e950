"""CPU oracle for the TokenOTBlock steps either side of the balanced transport.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports it; only
``tests/`` (and the bench's CPU baseline leg) use it, as the checker.

Restates with differentiable torch ops (float64 on the CPU in the tests) what
vv137/deepfold-linear's TokenOTBlock.forward does around its transport,
src/deepfold/model/trunk_block.py:

* ``layer_norm``           -- nn.LayerNorm(d_model) (:66, :94): biased variance, eps 1e-5;
* ``sink_projections``     -- :165-175: h_s = ln_sink(h); Q_s, K_s, V_s = h_s W^T viewed
                              (B, N, H, d) -> (B, H, N, d); Q_s, K_s = F.normalize(., dim=-1)
                              (division by max(|u|, 1e-12));
* ``gated_coordinate_update`` -- :189-204: vec = x_c - x; gate = sigmoid(w_gate . ln_gate(h)
                              + b); lam = tanh(lambda_raw) / H; x + mask * gate * sum_h lam_h vec_h;
* ``transport_step``       -- :165-204 chained with the oracle balanced transport
                              (oracle/balanced_transport.py) and w_o_sink.

Pinned by tests/test_oracle_trunk.py: the LayerNorm against torch's
``F.layer_norm`` and the head normalisation against ``F.normalize`` (library
routines); unit head norms; the eps branch on a zero row; the coordinate update's
closed forms (gate 1/2 at zero gate weights, lambda = tanh^-1 chosen values, mask 0
leaves x unchanged, one head moves x towards x_c by lam * gate); gradcheck in
float64.
"""

from __future__ import annotations

import torch

from oracle import balanced_transport as bt


def layer_norm(x, w, b, eps=1e-5):
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * w + b


def _head_normalize(u, eps=1e-12):
    return u / u.norm(dim=-1, keepdim=True).clamp(min=eps)


def sink_projections(h, ln_w, ln_b, w_q, w_k, w_v, n_heads):
    """h (B, N, C) -> Q_s, K_s, V_s (B, H, N, C/H); V_s None without w_v."""
    B, N, C = h.shape
    H = n_heads
    hs = layer_norm(h, ln_w, ln_b)
    heads = lambda u: u.reshape(B, N, H, C // H).permute(0, 2, 1, 3)
    q = _head_normalize(heads(hs @ w_q.transpose(0, 1)))
    k = _head_normalize(heads(hs @ w_k.transpose(0, 1)))
    v = None if w_v is None else heads(hs @ w_v.transpose(0, 1))
    return q, k, v


def gated_coordinate_update(h, x_res, x_centroid, ln_w, ln_b, w_gate, b_gate, lambda_raw, mask=None):
    """h (B, N, C), x_res (B, N, 3), x_centroid (B, H, N, 3) -> (B, N, 3)."""
    B, H = x_centroid.shape[:2]
    vec = x_centroid - x_res.unsqueeze(1)
    z = layer_norm(h, ln_w, ln_b) @ w_gate.reshape(-1, 1) + b_gate.reshape(1)
    gate = torch.sigmoid(z)  # (B, N, 1)
    lam = torch.tanh(lambda_raw).view(1, H, 1, 1) / H
    upd = gate * (lam * vec).sum(dim=1)
    if mask is not None:
        upd = upd * mask.unsqueeze(-1)
    return x_res + upd


def transport_step(params, h, x_res, mask, n_heads, K_iter=20):
    """trunk_block.py:165-204 with the oracle transport (feature transport on)."""
    B, N, C = h.shape
    q, k, v = sink_projections(h, params["ln_sink_w"], params["ln_sink_b"], params["w_q"], params["w_k"],
                               params["w_v"], n_heads)
    xc, hc = bt.balanced_transport_dual(q, k, x_res, v, params["eps"], params["alpha_h"], params["r_h"],
                                        K_iter=K_iter, mask=mask)
    h = h + (hc.permute(0, 2, 1, 3).reshape(B, N, C) @ params["w_o"].transpose(0, 1)) * mask.unsqueeze(-1)
    x = gated_coordinate_update(h, x_res, xc, params["ln_gate_w"], params["ln_gate_b"], params["w_gate"],
                                params["b_gate"], params["lambda_raw"], mask)
    return h, x
