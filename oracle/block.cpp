// oracle: one DiT block forward and backward — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Restates dit_block (src/dit.h:164-266) with autodiff_safe semantics, batch-major tokens:
//   ssg_b = ssg + gcond[b] = [sc_a | sh_a | g_a | sc_f | sh_f | g_f]
//   h   = rms(x) * pre_g * (1 + sc_a) + sh_a                    (rms_norm eps norm_eps, src/nn.h:40)
//   qkv = dit_lin(h); q,k,qd,kd = rope(rms_head(., q/k gamma, qk_eps)); v    (src/dit.h:208-217)
//   x1  = x + dit_lin(diff_attn(q,k,v,qd,kd)) * sigmoid(1 - g_a)              (src/dit.h:222-223)
//   hc  = rms(x1) * cross_g; cq,cqd = rms_head(dit_lin(hc)); ck,ckd,cv from dit_lin(context)
//   x2  = x1 + dit_lin(diff_attn(cq,ck,cv,cqd,ckd))                           (src/dit.h:226-242)
//         [+ ladd: the inpaint local add, zero on the memory rows                (src/dit.h:244-254)]
//   f   = rms(x2) * ff_g * (1 + sc_f) + sh_f; f = dit_lin(f) + b; f = val * silu(glu)
//   out = x2 + (dit_lin(f) + b) * sigmoid(1 - g_f)                            (src/dit.h:257-265)
// RoPE is ggml's NEOX mode on the first rope_dims of each head, positions 0..S-1, theta_i =
// pos * base^(-2i/rope_dims), pairs (i, i + rope_dims/2) (src/nn.h:53-59). Backward: hand-derived
// VJP of every op; the linears and attention reuse the closed forms of dit_lin.cpp / attn.cpp.
// Pinned by torch float64 autograd vectors (tests/golden/dit_block_autograd.npz).
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace {

using dvec = std::vector<double>;

struct Cfg {
    int B, S, Ctx, dim, H, HDm, inner, rope, window;
    double base, eps, qk_eps;
};

dvec fv(const float* p, size_t n) { return dvec(p, p + n); }
std::vector<float> tof(const dvec& v) { return std::vector<float>(v.begin(), v.end()); }

// ---- dit_lin through the float oracle entry points (double inside, float boundary)
struct Lin {
    const float *W, *b, *A, *Bm, *mag, *bnsq;
    int in, out, r;
    float s;
    int dora;
};

dvec lin_fwd(const Lin& L, const dvec& X, int N) {
    std::vector<float> xf = tof(X), y((size_t)N * L.out);
    orc_dit_lin_fwd(xf.data(), N, L.W, L.in, L.out, L.A, L.Bm, L.r, L.s, L.dora, L.mag, L.bnsq, L.b, y.data(),
                    nullptr, nullptr, nullptr);
    return dvec(y.begin(), y.end());
}

dvec lin_bwd(const Lin& L, const dvec& X, int N, const dvec& dY, float* dA, float* dB, float* dm) {
    std::vector<float> xf = tof(X), dyf = tof(dY), dx((size_t)N * L.in);
    std::vector<float> a((size_t)L.r * L.in), b((size_t)L.out * L.r), m((size_t)L.out);
    orc_dit_lin_bwd(xf.data(), N, L.W, L.in, L.out, L.A, L.Bm, L.r, L.s, L.dora, L.mag, L.bnsq, dyf.data(), dx.data(),
                    L.r ? a.data() : nullptr, L.r ? b.data() : nullptr, m.data());
    if (L.r) {
        for (size_t i = 0; i < a.size(); ++i) dA[i] += a[i];
        for (size_t i = 0; i < b.size(); ++i) dB[i] += b[i];
        if (L.dora && dm)
            for (size_t i = 0; i < m.size(); ++i) dm[i] += m[i];
    }
    return dvec(dx.begin(), dx.end());
}

// ---- rms norm over rows of width w: y = x * rstd * gamma
void rms_fwd(const dvec& x, int n, int w, const float* g, double eps, dvec& y, dvec& rstd) {
    y.resize((size_t)n * w);
    rstd.resize((size_t)n);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        double ss = 0;
        for (int j = 0; j < w; ++j) ss += x[(size_t)i * w + j] * x[(size_t)i * w + j];
        const double r = 1.0 / std::sqrt(ss / w + eps);
        rstd[(size_t)i] = r;
        for (int j = 0; j < w; ++j) y[(size_t)i * w + j] = x[(size_t)i * w + j] * r * (g ? g[j] : 1.0);
    }
}
// dx from dy for y = x * rstd * gamma
void rms_bwd(const dvec& x, const dvec& rstd, int n, int w, const float* g, const dvec& dy, dvec& dx) {
    dx.assign((size_t)n * w, 0.0);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        const double r = rstd[(size_t)i];
        double dot = 0;
        for (int j = 0; j < w; ++j) dot += dy[(size_t)i * w + j] * (g ? g[j] : 1.0) * x[(size_t)i * w + j];
        for (int j = 0; j < w; ++j) {
            const double gj = g ? g[j] : 1.0;
            dx[(size_t)i * w + j] = r * dy[(size_t)i * w + j] * gj - r * r * r * x[(size_t)i * w + j] * dot / w;
        }
    }
}

// NEOX rotary on a 64-vector's first `rope` dims
void rope_vec(double* v, int rope, double pos, double base, bool inverse) {
    const int half = rope / 2;
    for (int i = 0; i < half; ++i) {
        const double th = pos * std::pow(base, -2.0 * i / rope);
        const double c = std::cos(th), s = inverse ? -std::sin(th) : std::sin(th);
        const double a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
    }
}

double sigm(double z) { return 1.0 / (1.0 + std::exp(-z)); }

struct Fwd {
    dvec x, h, rs_a, hn_a, qkv, q, k, v, qd, kd, rq[4], pre[4], o, y, x1, rs_c, hc, qf, kv, cq, ck, cv, cqd, ckd,
        rcq[2], rck[2], cpre[4], oc, x2, rs_f, fn, f_in, F, g, yf, out;
    std::vector<float> lse;
};

// heads: take column block `part` (width dim) of a [n][parts*dim] matrix -> [B*H][Sx][64]
dvec heads(const dvec& m, int B, int Sx, int parts, int part, int dim, int H) {
    dvec o((size_t)B * H * Sx * 64);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < Sx; ++t)
            for (int hh = 0; hh < H; ++hh)
                for (int d = 0; d < 64; ++d)
                    o[(((size_t)b * H + hh) * Sx + t) * 64 + d] =
                        m[((size_t)b * Sx + t) * parts * dim + (size_t)part * dim + hh * 64 + d];
    return o;
}
void unheads_add(const dvec& hv, int B, int Sx, int parts, int part, int dim, int H, dvec& m) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < Sx; ++t)
            for (int hh = 0; hh < H; ++hh)
                for (int d = 0; d < 64; ++d)
                    m[((size_t)b * Sx + t) * parts * dim + (size_t)part * dim + hh * 64 + d] +=
                        hv[(((size_t)b * H + hh) * Sx + t) * 64 + d];
}

// per-head rms norm (over 64) then optional rope; pre = normalised (before gamma) for backward
void qk_fwd(dvec& hv, int BH, int Sx, const float* g, double eps, int rope, double base, dvec& rstd) {
    rstd.resize((size_t)BH * Sx);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < BH * Sx; ++i) {
        double* p = &hv[(size_t)i * 64];
        double ss = 0;
        for (int d = 0; d < 64; ++d) ss += p[d] * p[d];
        const double r = 1.0 / std::sqrt(ss / 64 + eps);
        rstd[(size_t)i] = r;
        for (int d = 0; d < 64; ++d) p[d] = p[d] * r * g[d];
        if (rope) rope_vec(p, rope, (double)(i % Sx), base, false);
    }
}
// backward of qk_fwd given the pre-norm input `in`
dvec qk_bwd(const dvec& in, const dvec& rstd, int BH, int Sx, const float* g, int rope, double base, dvec dy) {
    dvec dx((size_t)BH * Sx * 64);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < BH * Sx; ++i) {
        double* d = &dy[(size_t)i * 64];
        if (rope) rope_vec(d, rope, (double)(i % Sx), base, true);   // rotation transpose
        const double r = rstd[(size_t)i];
        const double* x = &in[(size_t)i * 64];
        double dot = 0;
        for (int j = 0; j < 64; ++j) dot += d[j] * g[j] * x[j];
        for (int j = 0; j < 64; ++j) dx[(size_t)i * 64 + j] = r * d[j] * g[j] - r * r * r * x[j] * dot / 64;
    }
    return dx;
}

dvec attn_fwd(const dvec& q1, const dvec& k1, const dvec& q2, const dvec& k2, const dvec& v, int BH, int Sq, int Sk,
              int window) {
    std::vector<float> a = tof(q1), b = tof(k1), c = tof(q2), d = tof(k2), e = tof(v), o((size_t)BH * Sq * 64);
    orc_diff_attn_fwd(a.data(), b.data(), c.data(), d.data(), e.data(), BH, Sq, Sk, 64, 0.125f, window, o.data(),
                      nullptr, nullptr, nullptr, nullptr);
    return dvec(o.begin(), o.end());
}

// [B*H][S][64] -> token-major [B*S][H*64]
dvec tokmajor(const dvec& hv, int B, int H, int Sx) {
    dvec o((size_t)B * Sx * H * 64);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh)
            for (int t = 0; t < Sx; ++t)
                for (int d = 0; d < 64; ++d)
                    o[((size_t)b * Sx + t) * H * 64 + hh * 64 + d] = hv[(((size_t)b * H + hh) * Sx + t) * 64 + d];
    return o;
}
dvec headmajor(const dvec& tm, int B, int H, int Sx) {
    dvec o((size_t)B * H * Sx * 64);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh)
            for (int t = 0; t < Sx; ++t)
                for (int d = 0; d < 64; ++d)
                    o[(((size_t)b * H + hh) * Sx + t) * 64 + d] = tm[((size_t)b * Sx + t) * H * 64 + hh * 64 + d];
    return o;
}

}  // namespace

extern "C" {

static Lin mk(const orc_block* p, int t) {
    const int dim = p->dim;
    const int ins[7] = {dim, dim, dim, dim, dim, dim, p->inner};
    const int outs[7] = {5 * dim, dim, 2 * dim, 3 * dim, dim, 2 * p->inner, dim};
    return Lin{p->W[t], p->bias[t], p->A[t], p->Bm[t], p->mag[t], p->bnsq[t], ins[t], outs[t], p->rank, p->scale,
               p->dora};
}

static void block_forward(const orc_block* p, const float* xin, const float* ctxin, const float* gc, Fwd& f) {
    const int B = p->B, S = p->S, Ctx = p->Ctx, dim = p->dim, H = p->heads, N = B * S, NC = B * Ctx;
    const double eps = p->norm_eps, qe = p->qk_eps, base = p->rope_base;
    f.x = fv(xin, (size_t)N * dim);
    auto mod = [&](int b, int part, int c) { return (double)p->ssg[part * dim + c] + gc[(size_t)b * 6 * dim + part * dim + c]; };
    // self attention
    rms_fwd(f.x, N, dim, p->pre_g, eps, f.hn_a, f.rs_a);
    f.h.resize((size_t)N * dim);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < dim; ++c)
            f.h[(size_t)n * dim + c] = f.hn_a[(size_t)n * dim + c] * (1 + mod(n / S, 0, c)) + mod(n / S, 1, c);
    f.qkv = lin_fwd(mk(p, 0), f.h, N);
    const dvec* src = &f.qkv;
    dvec* dst[5] = {&f.q, &f.k, &f.v, &f.qd, &f.kd};
    for (int i = 0; i < 5; ++i) *dst[i] = heads(*src, B, S, 5, i, dim, H);
    f.pre[0] = f.q; f.pre[1] = f.k; f.pre[2] = f.qd; f.pre[3] = f.kd;
    qk_fwd(f.q, B * H, S, p->sq_g, qe, p->rope_dims, base, f.rq[0]);
    qk_fwd(f.k, B * H, S, p->sk_g, qe, p->rope_dims, base, f.rq[1]);
    qk_fwd(f.qd, B * H, S, p->sq_g, qe, p->rope_dims, base, f.rq[2]);
    qk_fwd(f.kd, B * H, S, p->sk_g, qe, p->rope_dims, base, f.rq[3]);
    f.o = tokmajor(attn_fwd(f.q, f.k, f.qd, f.kd, f.v, B * H, S, S, p->window), B, H, S);
    f.y = lin_fwd(mk(p, 1), f.o, N);
    f.x1.resize((size_t)N * dim);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < dim; ++c)
            f.x1[(size_t)n * dim + c] = f.x[(size_t)n * dim + c] + f.y[(size_t)n * dim + c] * sigm(1 - mod(n / S, 2, c));
    // cross attention
    rms_fwd(f.x1, N, dim, p->cross_g, eps, f.hc, f.rs_c);
    f.qf = lin_fwd(mk(p, 2), f.hc, N);
    f.kv = lin_fwd(mk(p, 3), fv(ctxin, (size_t)NC * dim), NC);
    f.cq = heads(f.qf, B, S, 2, 0, dim, H);
    f.cqd = heads(f.qf, B, S, 2, 1, dim, H);
    f.ck = heads(f.kv, B, Ctx, 3, 0, dim, H);
    f.ckd = heads(f.kv, B, Ctx, 3, 1, dim, H);
    f.cv = heads(f.kv, B, Ctx, 3, 2, dim, H);
    f.cpre[0] = f.cq; f.cpre[1] = f.ck; f.cpre[2] = f.cqd; f.cpre[3] = f.ckd;
    qk_fwd(f.cq, B * H, S, p->cq_g, qe, 0, base, f.rcq[0]);
    qk_fwd(f.cqd, B * H, S, p->cq_g, qe, 0, base, f.rcq[1]);
    qk_fwd(f.ck, B * H, Ctx, p->ck_g, qe, 0, base, f.rck[0]);
    qk_fwd(f.ckd, B * H, Ctx, p->ck_g, qe, 0, base, f.rck[1]);
    f.oc = tokmajor(attn_fwd(f.cq, f.ck, f.cqd, f.ckd, f.cv, B * H, S, Ctx, 0), B, H, S);
    const dvec yc = lin_fwd(mk(p, 4), f.oc, N);
    f.x2.resize((size_t)N * dim);
    for (size_t i = 0; i < f.x2.size(); ++i) f.x2[i] = f.x1[i] + yc[i];
    if (p->ladd)
        for (size_t i = 0; i < f.x2.size(); ++i) f.x2[i] += (double)p->ladd[i];
    // feed-forward
    rms_fwd(f.x2, N, dim, p->ff_g, eps, f.fn, f.rs_f);
    f.f_in.resize((size_t)N * dim);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < dim; ++c)
            f.f_in[(size_t)n * dim + c] = f.fn[(size_t)n * dim + c] * (1 + mod(n / S, 3, c)) + mod(n / S, 4, c);
    f.F = lin_fwd(mk(p, 5), f.f_in, N);
    const int I = p->inner;
    f.g.resize((size_t)N * I);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < I; ++c) {
            const double val = f.F[(size_t)n * 2 * I + c], glu = f.F[(size_t)n * 2 * I + I + c];
            f.g[(size_t)n * I + c] = val * glu * sigm(glu);
        }
    f.yf = lin_fwd(mk(p, 6), f.g, N);
    f.out.resize((size_t)N * dim);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < dim; ++c)
            f.out[(size_t)n * dim + c] = f.x2[(size_t)n * dim + c] + f.yf[(size_t)n * dim + c] * sigm(1 - mod(n / S, 5, c));
}

void orc_block_fwd(const orc_block* p, const float* x, const float* ctx, const float* gcond, float* out) {
    Fwd f;
    block_forward(p, x, ctx, gcond, f);
    for (size_t i = 0; i < f.out.size(); ++i) out[i] = (float)f.out[i];
}

// dA[t] [rank][in], dB[t] [out][rank], dm[t] [out] accumulate (+=); dx, dctx, dgcond are written.
void orc_block_bwd(const orc_block* p, const float* x, const float* ctxin, const float* gc, const float* dout,
                   float* dx, float* dctx, float* dgcond, float* const* dA, float* const* dB, float* const* dm) {
    Fwd f;
    block_forward(p, x, ctxin, gc, f);
    const int B = p->B, S = p->S, Ctx = p->Ctx, dim = p->dim, H = p->heads, N = B * S, NC = B * Ctx, I = p->inner;
    const double base = p->rope_base;
    auto mod = [&](int b, int part, int c) { return (double)p->ssg[part * dim + c] + gc[(size_t)b * 6 * dim + part * dim + c]; };
    dvec dssg((size_t)B * 6 * dim, 0.0);
    auto dmod = [&](int b, int part, int c) -> double& { return dssg[(size_t)b * 6 * dim + part * dim + c]; };
    dvec d3 = fv(dout, (size_t)N * dim);
    // out = x2 + yf * s_f
    dvec dyf((size_t)N * dim), dx2 = d3;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < dim; ++c)
        for (int n = 0; n < N; ++n) {
            const size_t i = (size_t)n * dim + c;
            const double s = sigm(1 - mod(n / S, 5, c));
            dyf[i] = d3[i] * s;
            dmod(n / S, 5, c) += -d3[i] * f.yf[i] * s * (1 - s);
        }
    const dvec dg = lin_bwd(mk(p, 6), f.g, N, dyf, dA[6], dB[6], dm[6]);
    dvec dF((size_t)N * 2 * I);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int c = 0; c < I; ++c) {
            const double val = f.F[(size_t)n * 2 * I + c], glu = f.F[(size_t)n * 2 * I + I + c];
            const double sg = sigm(glu), d = dg[(size_t)n * I + c];
            dF[(size_t)n * 2 * I + c] = d * glu * sg;
            dF[(size_t)n * 2 * I + I + c] = d * val * (sg + glu * sg * (1 - sg));
        }
    const dvec dfin = lin_bwd(mk(p, 5), f.f_in, N, dF, dA[5], dB[5], dm[5]);
    dvec dfn((size_t)N * dim);
#pragma omp parallel for schedule(static)
    for (int c = 0; c < dim; ++c)
        for (int n = 0; n < N; ++n) {
            const size_t i = (size_t)n * dim + c;
            dfn[i] = dfin[i] * (1 + mod(n / S, 3, c));
            dmod(n / S, 3, c) += dfin[i] * f.fn[i];
            dmod(n / S, 4, c) += dfin[i];
        }
    dvec t;
    rms_bwd(f.x2, f.rs_f, N, dim, p->ff_g, dfn, t);
    for (size_t i = 0; i < dx2.size(); ++i) dx2[i] += t[i];
    if (p->dladd)   // x2 = x1 + yc + ladd: the local add receives dx2
        for (size_t i = 0; i < dx2.size(); ++i) p->dladd[i] = (float)dx2[i];
    // x2 = x1 + yc
    dvec dx1 = dx2;
    const dvec doc = lin_bwd(mk(p, 4), f.oc, N, dx2, dA[4], dB[4], dm[4]);
    // cross attention backward
    {
        std::vector<float> a = tof(f.cq), b = tof(f.ck), c2 = tof(f.cqd), d = tof(f.ckd), e = tof(f.cv),
                           g = tof(headmajor(doc, B, H, S));
        std::vector<float> dq1(a.size()), dk1(b.size()), dq2(a.size()), dk2(b.size()), dv(b.size());
        orc_diff_attn_bwd(a.data(), b.data(), c2.data(), d.data(), e.data(), g.data(), B * H, S, Ctx, 64, 0.125f, 0,
                          dq1.data(), dk1.data(), dq2.data(), dk2.data(), dv.data());
        dvec dqf((size_t)N * 2 * dim, 0.0), dkv((size_t)NC * 3 * dim, 0.0);
        unheads_add(qk_bwd(f.cpre[0], f.rcq[0], B * H, S, p->cq_g, 0, base, dvec(dq1.begin(), dq1.end())), B, S, 2, 0, dim, H, dqf);
        unheads_add(qk_bwd(f.cpre[2], f.rcq[1], B * H, S, p->cq_g, 0, base, dvec(dq2.begin(), dq2.end())), B, S, 2, 1, dim, H, dqf);
        unheads_add(qk_bwd(f.cpre[1], f.rck[0], B * H, Ctx, p->ck_g, 0, base, dvec(dk1.begin(), dk1.end())), B, Ctx, 3, 0, dim, H, dkv);
        unheads_add(qk_bwd(f.cpre[3], f.rck[1], B * H, Ctx, p->ck_g, 0, base, dvec(dk2.begin(), dk2.end())), B, Ctx, 3, 1, dim, H, dkv);
        unheads_add(dvec(dv.begin(), dv.end()), B, Ctx, 3, 2, dim, H, dkv);
        const dvec dhc = lin_bwd(mk(p, 2), f.hc, N, dqf, dA[2], dB[2], dm[2]);
        const dvec dc = lin_bwd(mk(p, 3), fv(ctxin, (size_t)NC * dim), NC, dkv, dA[3], dB[3], dm[3]);
        for (size_t i = 0; i < dc.size(); ++i) dctx[i] = (float)dc[i];
        rms_bwd(f.x1, f.rs_c, N, dim, p->cross_g, dhc, t);
        for (size_t i = 0; i < dx1.size(); ++i) dx1[i] += t[i];
    }
    // x1 = x + y * s_a
    dvec dy((size_t)N * dim), dxx = dx1;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < dim; ++c)
        for (int n = 0; n < N; ++n) {
            const size_t i = (size_t)n * dim + c;
            const double s = sigm(1 - mod(n / S, 2, c));
            dy[i] = dx1[i] * s;
            dmod(n / S, 2, c) += -dx1[i] * f.y[i] * s * (1 - s);
        }
    const dvec dob = lin_bwd(mk(p, 1), f.o, N, dy, dA[1], dB[1], dm[1]);
    {
        std::vector<float> a = tof(f.q), b = tof(f.k), c2 = tof(f.qd), d = tof(f.kd), e = tof(f.v),
                           g = tof(headmajor(dob, B, H, S));
        std::vector<float> dq1(a.size()), dk1(a.size()), dq2(a.size()), dk2(a.size()), dv(a.size());
        orc_diff_attn_bwd(a.data(), b.data(), c2.data(), d.data(), e.data(), g.data(), B * H, S, S, 64, 0.125f,
                          p->window, dq1.data(), dk1.data(), dq2.data(), dk2.data(), dv.data());
        dvec dqkv((size_t)N * 5 * dim, 0.0);
        unheads_add(qk_bwd(f.pre[0], f.rq[0], B * H, S, p->sq_g, p->rope_dims, base, dvec(dq1.begin(), dq1.end())), B, S, 5, 0, dim, H, dqkv);
        unheads_add(qk_bwd(f.pre[1], f.rq[1], B * H, S, p->sk_g, p->rope_dims, base, dvec(dk1.begin(), dk1.end())), B, S, 5, 1, dim, H, dqkv);
        unheads_add(dvec(dv.begin(), dv.end()), B, S, 5, 2, dim, H, dqkv);
        unheads_add(qk_bwd(f.pre[2], f.rq[2], B * H, S, p->sq_g, p->rope_dims, base, dvec(dq2.begin(), dq2.end())), B, S, 5, 3, dim, H, dqkv);
        unheads_add(qk_bwd(f.pre[3], f.rq[3], B * H, S, p->sk_g, p->rope_dims, base, dvec(dk2.begin(), dk2.end())), B, S, 5, 4, dim, H, dqkv);
        const dvec dh = lin_bwd(mk(p, 0), f.h, N, dqkv, dA[0], dB[0], dm[0]);
        dvec dhn((size_t)N * dim);
#pragma omp parallel for schedule(static)
        for (int c = 0; c < dim; ++c)
            for (int n = 0; n < N; ++n) {
                const size_t i = (size_t)n * dim + c;
                dhn[i] = dh[i] * (1 + mod(n / S, 0, c));
                dmod(n / S, 0, c) += dh[i] * f.hn_a[i];
                dmod(n / S, 1, c) += dh[i];
            }
        rms_bwd(f.x, f.rs_a, N, dim, p->pre_g, dhn, t);
        for (size_t i = 0; i < dxx.size(); ++i) dxx[i] += t[i];
    }
    for (size_t i = 0; i < dxx.size(); ++i) dx[i] = (float)dxx[i];
    for (size_t i = 0; i < dssg.size(); ++i) dgcond[i] = (float)dssg[i];
}

}  // extern "C"

// exported for the oracle's own tests: rope_vec over n head vectors of 64 floats at positions pos[j]
extern "C" void orc_rope_neox(float* v, int n, int rope, const float* pos, float base) {
    for (int j = 0; j < n; ++j) {
        double d[64];
        for (int e = 0; e < 64; ++e) d[e] = v[64 * j + e];
        rope_vec(d, rope, (double)pos[j], (double)base, false);
        for (int e = 0; e < 64; ++e) v[64 * j + e] = (float)d[e];
    }
}
