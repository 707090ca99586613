"""QSF files of several shapes for the container tests (test helper):
a dense model with per-tensor type overrides, FP16 vectors and a separate
output head; the same with a tied head; a 2-bit + outlier model whose
embedding is in the model's type; an MoE layer of MXFP4 experts with
biases and a router."""
from __future__ import annotations

import numpy as np

from qstream_amd import qsf_format as F


def _vec(rng, n):
    return F.gaussian(rng, n).astype(np.float16).tobytes()


def dense(rng, tied=False, hidden=256, vocab=300, inter=512, bs=64):
    q = lambda qt, r, c: F.quantize_matrix(  # noqa: E731
        F.heavy_tail_weights(rng, r, c) if qt in (F.Q2_OUTLIER, F.Q4_OUTLIER) else F.gaussian(rng, (r, c), 0.02),
        qt, bs)
    layers = []
    for _ in range(3):
        layers.append([(F.T_ATTN_NORM_W, F.FP16, 1, hidden, _vec(rng, hidden)),
                       (F.T_ATTN_Q, 0xFF, hidden, hidden, q(F.Q4, hidden, hidden)),
                       (F.T_ATTN_K, F.Q4SYM, 128, hidden, q(F.Q4SYM, 128, hidden)),
                       (F.T_ATTN_V, F.Q2, 128, hidden, q(F.Q2, 128, hidden)),
                       (F.T_ATTN_O, F.Q4_OUTLIER, hidden, hidden, q(F.Q4_OUTLIER, hidden, hidden)),
                       (F.T_FFN_NORM_W, F.FP16, 1, hidden, _vec(rng, hidden)),
                       (F.T_FFN_GATE, F.Q2_OUTLIER, inter, hidden, q(F.Q2_OUTLIER, inter, hidden)),
                       (F.T_FFN_UP, F.Q3, inter, hidden, q(F.Q3, inter, hidden)),
                       (F.T_FFN_DOWN, F.Q3, hidden, inter, q(F.Q3, hidden, inter))])
    return dict(hidden=hidden, heads=8, kv_heads=4, vocab=vocab, inter=inter, layers=layers,
                quant_type=F.Q4, block_size=bs, embedding=(F.Q4, q(F.Q4, vocab, hidden)),
                final_norm=F.gaussian(rng, hidden).astype(np.float16),
                output_head=None if tied else q(F.Q4, vocab, hidden), tied=tied,
                activation=2, norm_type=2, pos_enc=1, rope_theta=500000.0, eps=1e-6)


def outlier_tied(rng, hidden=256, vocab=260, bs=128):
    q9 = lambda r, c: F.quantize_matrix(F.heavy_tail_weights(rng, r, c), F.Q2_OUTLIER, bs)  # noqa: E731
    layers = [[(F.T_ATTN_NORM_W, F.FP16, 1, hidden, _vec(rng, hidden)),
               (F.T_ATTN_Q, 0xFF, hidden, hidden, q9(hidden, hidden)),
               (F.T_FFN_DOWN, 0xFF, hidden, 384, q9(hidden, 384))]]
    return dict(hidden=hidden, heads=4, vocab=vocab, inter=384, layers=layers, quant_type=F.Q2_OUTLIER,
                block_size=bs, embedding=(F.Q2_OUTLIER, q9(vocab, hidden)),
                final_norm=F.gaussian(rng, hidden).astype(np.float16), tied=True,
                activation=0, norm_type=0, pos_enc=1, rope_theta=10000.0, eps=1e-5)


def moe(rng, n_exp=4, hidden=256, eid=128, vocab=200, k=2):
    recs = [(F.T_ATTN_NORM_W, F.FP16, 1, hidden, _vec(rng, hidden)),
            (F.T_MOE_ROUTER, F.Q4, n_exp, hidden,
             F.quantize_matrix(F.gaussian(rng, (n_exp, hidden), 0.02), F.Q4, 64))]
    for e in range(n_exp):
        for role, rows, cols in (("gate", eid, hidden), ("up", eid, hidden), ("down", hidden, eid)):
            recs.append((F.t_moe(e, role), F.MXFP4, rows, cols, F.random_mxfp4(rng, rows, cols)))
            recs.append((F.t_moe(e, role, bias=True), F.FP16, 1, rows, _vec(rng, rows)))
    return dict(hidden=hidden, heads=4, vocab=vocab, inter=eid, layers=[recs, list(recs)], quant_type=F.Q4,
                block_size=64, ffn_type=F.FFN_MOE, num_experts=n_exp, num_active_experts=k,
                moe_norm_topk=1, expert_dim=eid,
                embedding=(F.Q4, F.quantize_matrix(F.gaussian(rng, (vocab, hidden), 0.02), F.Q4, 64)),
                final_norm=F.gaussian(rng, hidden).astype(np.float16), tied=True)


def all_models(seed=0):
    rng = np.random.default_rng(seed)
    return {"dense": dense(rng), "dense_tied": dense(rng, tied=True), "outlier_tied": outlier_tied(rng),
            "moe": moe(rng)}
