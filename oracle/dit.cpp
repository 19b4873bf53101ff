// oracle: the whole DiT training loss and its gradients — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Restates, batch-major and per sample exactly as the reference runs one sample per graph:
//   dit_head  (src/dit.h:286-312)  te = mlp(time_embed, expo_features(t)), g = mlp(global_embed,
//             glob) + te, gcond = mlp(gce, g), context = mlp(cond_embed, cross);
//             x = dit_lin(pre_conv, x_t) + x_t; x = dit_lin(proj_in, x); x0 = [memory tokens; x]
//             (mlp_silu, src/dit.h:269-274: lin -> silu -> lin, biases on time_embed and gce)
//   blocks    orc_block_fwd / orc_block_bwd (block.cpp) for l = 0..depth-1; with inpaint local
//             conditioning each block adds le = mlp(local, local_cond) (local.0 -> silu -> local.2,
//             both with biases) to its T latent rows after the cross-attention (src/dit.h:244-254)
//   dit_tail  (src/dit.h:316-325)  drop memory tokens, v = dit_lin(proj_out, x);
//             v = dit_lin(post_conv, v) + v
//   loss      sum((v - target)^2) / (io*T), or sum((v - target)^2 * w_frame) with a loss weight
//             (src/train_dit.h:174-184)
// The backward is the chain of the closed-form VJPs: the linears through orc_dit_lin_bwd, the
// blocks through orc_block_bwd, silu' = s(z)(1 + z(1 - s(z))).
// Pinned by torch float64 autograd of an independent torch restatement (tests/golden/
// dit_autograd.npz), every adapter gradient of a depth-2 model with all 12 head/tail targets.
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

using fvec = std::vector<float>;

struct L {
    const orc_lin* l;
    int rank, dora;
    float s;
    bool adapted() const { return l->A && l->B; }
};

fvec lin_fwd(const L& q, const fvec& X, int N) {
    fvec y((size_t)N * q.l->out);
    const int r = q.adapted() ? q.rank : 0;
    orc_dit_lin_fwd(X.data(), N, q.l->W, q.l->in, q.l->out, r ? q.l->A : nullptr, r ? q.l->B : nullptr, r, q.s,
                    r ? q.dora : 0, q.l->mag, q.l->bnsq, q.l->bias, y.data(), nullptr, nullptr, nullptr);
    return y;
}

// dX (nullable) written; adapter gradients added
void lin_bwd(const L& q, const fvec& X, int N, const fvec& dY, float* dX, float* dA, float* dB, float* dm) {
    const int r = q.adapted() ? q.rank : 0;
    if (!r) {
        if (dX) orc_dit_lin_bwd(X.data(), N, q.l->W, q.l->in, q.l->out, nullptr, nullptr, 0, q.s, 0, nullptr, nullptr,
                                dY.data(), dX, nullptr, nullptr, nullptr);
        return;
    }
    fvec a((size_t)r * q.l->in), b((size_t)q.l->out * r), m((size_t)q.l->out);
    orc_dit_lin_bwd(X.data(), N, q.l->W, q.l->in, q.l->out, q.l->A, q.l->B, r, q.s, q.dora, q.l->mag, q.l->bnsq,
                    dY.data(), dX, a.data(), b.data(), m.data());
    for (size_t i = 0; i < a.size(); ++i) dA[i] += a[i];
    for (size_t i = 0; i < b.size(); ++i) dB[i] += b[i];
    if (q.dora && dm)
        for (size_t i = 0; i < m.size(); ++i) dm[i] += m[i];
}

double sig(double z) { return 1.0 / (1.0 + std::exp(-z)); }

struct Mlp {
    fvec h, a, y;   // pre-activation, silu(h), output
};

Mlp mlp_fwd(const L& l0, const L& l2, const fvec& x, int N) {
    Mlp m;
    m.h = lin_fwd(l0, x, N);
    m.a.resize(m.h.size());
    for (size_t i = 0; i < m.h.size(); ++i) m.a[i] = (float)(m.h[i] * sig(m.h[i]));
    m.y = lin_fwd(l2, m.a, N);
    return m;
}

// backward of mlp from dy; dx (nullable) written
void mlp_bwd(const L& l0, const L& l2, const Mlp& m, const fvec& x, int N, const fvec& dy, float* dx,
             float* const* dA, float* const* dB, float* const* dm, int i0, int i2) {
    fvec da(m.a.size());
    lin_bwd(l2, m.a, N, dy, da.data(), dA[i2], dB[i2], dm[i2]);
    fvec dh(m.h.size());
    for (size_t i = 0; i < dh.size(); ++i) {
        const double z = m.h[i], sz = sig(z);
        dh[i] = (float)(da[i] * sz * (1.0 + z * (1.0 - sz)));
    }
    lin_bwd(l0, x, N, dh, dx, dA[i0], dB[i0], dm[i0]);
}

}  // namespace

extern "C" {

void orc_expo_features(float t, float* out, int dim, float min_f, float max_f) {
    const int half = dim / 2;
    const float lmin = logf(min_f), lmax = logf(max_f), two_pi = 6.28318530717958648f;
    for (int i = 0; i < half; ++i) {
        const float ramp = half > 1 ? (float)i / (float)(half - 1) : 0.0f;
        const float f = expf(ramp * (lmax - lmin) + lmin);
        const float arg = t * f * two_pi;
        out[i] = cosf(arg);
        out[half + i] = sinf(arg);
    }
}

void orc_dit_loss(const orc_dit* p, const float* x_t, const float* target, const float* t, const float* cross,
                  const float* glob, const float* loss_weight, float* velocity, double* loss,
                  float* const* dA_blocks, float* const* dB_blocks, float* const* dm_blocks,
                  float* const* dA_head, float* const* dB_head, float* const* dm_head,
                  float* const* dA_local, float* const* dB_local, float* const* dm_local) {
    const int B = p->B, T = p->T, Ctx = p->Ctx, io = p->io, dim = p->dim, mem = p->mem, S = mem + T;
    const bool grad = dA_blocks != nullptr;
    const bool local = p->local_dim > 0 && p->local && p->local_cond;
    auto hl = [&](int i) { return L{&p->head[i], p->rank, p->dora, p->scale}; };
    auto ll = [&](int l, int k) { return L{&p->local[2 * l + k], p->rank, p->dora, p->scale}; };
    std::vector<float*> dAl((size_t)2 * p->depth, nullptr), dBl = dAl, dml = dAl;
    if (grad && local)
        for (size_t i = 0; i < dAl.size(); ++i) {
            dAl[i] = dA_local ? dA_local[i] : nullptr;
            dBl[i] = dB_local ? dB_local[i] : nullptr;
            dml[i] = dm_local ? dm_local[i] : nullptr;
        }
    float* const* dAh = dA_head;
    float* const* dBh = dB_head;
    std::vector<float*> dmh_v(ORC_NHEAD, nullptr), dmb_v((size_t)7 * p->depth, nullptr);
    if (grad) {
        for (int i = 0; i < ORC_NHEAD; ++i) dmh_v[i] = dm_head ? dm_head[i] : nullptr;
        for (size_t i = 0; i < dmb_v.size(); ++i) dmb_v[i] = dm_blocks ? dm_blocks[i] : nullptr;
    }
    for (int b = 0; b < B; ++b) {
        // ---- head
        fvec tf(p->time_dim);
        orc_expo_features(t[b], tf.data(), p->time_dim, p->time_min_freq, p->time_max_freq);
        const Mlp te = mlp_fwd(hl(ORC_TIME0), hl(ORC_TIME2), tf, 1);
        const fvec gl(glob + (size_t)b * p->cond_dim, glob + (size_t)(b + 1) * p->cond_dim);
        const Mlp ge = mlp_fwd(hl(ORC_GLOBAL0), hl(ORC_GLOBAL2), gl, 1);
        fvec g(dim);
        for (int c = 0; c < dim; ++c) g[c] = ge.y[c] + te.y[c];
        const Mlp gc = mlp_fwd(hl(ORC_GCE0), hl(ORC_GCE2), g, 1);
        const fvec cr(cross + (size_t)b * Ctx * p->cond_dim, cross + (size_t)(b + 1) * Ctx * p->cond_dim);
        const Mlp ce = mlp_fwd(hl(ORC_COND0), hl(ORC_COND2), cr, Ctx);
        const fvec xin(x_t + (size_t)b * T * io, x_t + (size_t)(b + 1) * T * io);
        fvec xp = lin_fwd(hl(ORC_PRE_CONV), xin, T);
        for (size_t i = 0; i < xp.size(); ++i) xp[i] += xin[i];
        const fvec xi = lin_fwd(hl(ORC_PROJ_IN), xp, T);
        std::vector<fvec> xs(p->depth + 1, fvec((size_t)S * dim));
        std::memcpy(xs[0].data(), p->memory_tokens, sizeof(float) * mem * dim);
        std::memcpy(xs[0].data() + (size_t)mem * dim, xi.data(), sizeof(float) * T * dim);
        // ---- blocks (with the local conditioning's per-block MLP, added to the latent rows)
        std::vector<orc_block> bl(p->depth);
        std::vector<Mlp> lm(local ? p->depth : 0);
        std::vector<fvec> ladd(local ? p->depth : 0), dladd(local ? p->depth : 0);
        fvec lc;
        if (local) lc.assign(p->local_cond + (size_t)b * T * p->local_dim, p->local_cond + (size_t)(b + 1) * T * p->local_dim);
        for (int l = 0; l < p->depth; ++l) {
            bl[l] = p->blocks[l];
            bl[l].B = 1; bl[l].S = S; bl[l].Ctx = Ctx; bl[l].dim = dim; bl[l].heads = p->heads;
            bl[l].inner = p->inner; bl[l].rope_dims = p->rope_dims; bl[l].window = p->window;
            bl[l].rope_base = p->rope_base; bl[l].norm_eps = p->norm_eps; bl[l].qk_eps = p->qk_eps;
            bl[l].rank = p->rank; bl[l].dora = p->dora; bl[l].scale = p->scale;
            bl[l].ladd = nullptr;
            bl[l].dladd = nullptr;
            if (local) {
                lm[l] = mlp_fwd(ll(l, 0), ll(l, 1), lc, T);
                ladd[l].assign((size_t)S * dim, 0.0f);
                std::memcpy(ladd[l].data() + (size_t)mem * dim, lm[l].y.data(), sizeof(float) * T * dim);
                dladd[l].resize((size_t)S * dim);
                bl[l].ladd = ladd[l].data();
                bl[l].dladd = dladd[l].data();
            }
            orc_block_fwd(&bl[l], xs[l].data(), ce.y.data(), gc.y.data(), xs[l + 1].data());
        }
        // ---- tail
        const fvec xt(xs[p->depth].begin() + (size_t)mem * dim, xs[p->depth].end());
        const fvec v0 = lin_fwd(hl(ORC_PROJ_OUT), xt, T);
        fvec v = lin_fwd(hl(ORC_POST_CONV), v0, T);
        for (size_t i = 0; i < v.size(); ++i) v[i] += v0[i];
        if (velocity) std::memcpy(velocity + (size_t)b * T * io, v.data(), sizeof(float) * T * io);
        double ls = 0.0;
        fvec dv((size_t)T * io);
        for (int f = 0; f < T; ++f) {
            const double w = loss_weight ? (double)loss_weight[(size_t)b * T + f] : 1.0 / ((double)io * T);
            for (int c = 0; c < io; ++c) {
                const size_t i = (size_t)f * io + c;
                const double d = (double)v[i] - target[(size_t)b * T * io + i];
                ls += d * d * w;
                dv[i] = (float)(2.0 * d * w);
            }
        }
        loss[b] = ls;
        if (!grad) continue;
        // ---- backward: tail
        fvec dv0 = dv, tmp((size_t)T * io);
        lin_bwd(hl(ORC_POST_CONV), v0, T, dv, tmp.data(), dAh[ORC_POST_CONV], dBh[ORC_POST_CONV], dmh_v[ORC_POST_CONV]);
        for (size_t i = 0; i < dv0.size(); ++i) dv0[i] += tmp[i];
        fvec dxt((size_t)T * dim);
        lin_bwd(hl(ORC_PROJ_OUT), xt, T, dv0, dxt.data(), dAh[ORC_PROJ_OUT], dBh[ORC_PROJ_OUT], dmh_v[ORC_PROJ_OUT]);
        fvec dx((size_t)S * dim, 0.0f), dxn((size_t)S * dim);
        std::memcpy(dx.data() + (size_t)mem * dim, dxt.data(), sizeof(float) * T * dim);
        // ---- blocks in reverse
        fvec dctx((size_t)Ctx * dim, 0.0f), dgc((size_t)6 * dim, 0.0f), tc((size_t)Ctx * dim), tg((size_t)6 * dim);
        for (int l = p->depth - 1; l >= 0; --l) {
            orc_block_bwd(&bl[l], xs[l].data(), ce.y.data(), gc.y.data(), dx.data(), dxn.data(), tc.data(), tg.data(),
                          dA_blocks + (size_t)l * 7, dB_blocks + (size_t)l * 7, dmb_v.data() + (size_t)l * 7);
            for (size_t i = 0; i < dctx.size(); ++i) dctx[i] += tc[i];
            for (size_t i = 0; i < dgc.size(); ++i) dgc[i] += tg[i];
            if (local) {   // le enters the latent rows: its gradient is dladd there
                const fvec dle(dladd[l].begin() + (size_t)mem * dim, dladd[l].end());
                mlp_bwd(ll(l, 0), ll(l, 1), lm[l], lc, T, dle, nullptr, dAl.data(), dBl.data(), dml.data(), 2 * l,
                        2 * l + 1);
            }
            dx.swap(dxn);
        }
        // ---- head backward
        fvec dxi(dx.begin() + (size_t)mem * dim, dx.end());
        fvec dxp((size_t)T * io);
        lin_bwd(hl(ORC_PROJ_IN), xp, T, dxi, dxp.data(), dAh[ORC_PROJ_IN], dBh[ORC_PROJ_IN], dmh_v[ORC_PROJ_IN]);
        lin_bwd(hl(ORC_PRE_CONV), xin, T, dxp, nullptr, dAh[ORC_PRE_CONV], dBh[ORC_PRE_CONV], dmh_v[ORC_PRE_CONV]);
        fvec dg(dim);
        mlp_bwd(hl(ORC_GCE0), hl(ORC_GCE2), gc, g, 1, dgc, dg.data(), dAh, dBh, dmh_v.data(), ORC_GCE0, ORC_GCE2);
        mlp_bwd(hl(ORC_GLOBAL0), hl(ORC_GLOBAL2), ge, gl, 1, dg, nullptr, dAh, dBh, dmh_v.data(), ORC_GLOBAL0,
                ORC_GLOBAL2);
        mlp_bwd(hl(ORC_TIME0), hl(ORC_TIME2), te, tf, 1, dg, nullptr, dAh, dBh, dmh_v.data(), ORC_TIME0, ORC_TIME2);
        mlp_bwd(hl(ORC_COND0), hl(ORC_COND2), ce, cr, Ctx, dctx, nullptr, dAh, dBh, dmh_v.data(), ORC_COND0,
                ORC_COND2);
    }
}

}  // extern "C"
