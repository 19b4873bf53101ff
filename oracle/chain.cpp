// oracle: composed adapter chains over a frozen base (inference) — TEST INFRASTRUCTURE ONLY.
//
// Two restatements of the reference, in double precision:
//  * the sequential merge that apply_loras performs for the lora / dora-rows families
//    (src/lora.h:111-143, graph path; the host path src/lora.h:146-222 is the same arithmetic):
//    per adapter in chain order (skipped when strength is 0), V = W + s B A with
//    s = (alpha / rank) * strength; lora: W = V; dora-rows: W = diag(m / sqrt(sum_in V^2 + in 1e-12)) V
//    (the graph path's rms_norm(V, 1e-12) / sqrt(in) times the magnitude);
//  * build_functional_lora's fold (src/lora.h:372-622) and the composed forward of dit_lin over it
//    (src/dit.h:108-117): y = c0 (.) (W x) + sum_k s_k B'_k (A_k x), where walking the chain, each
//    dora adapter j multiplies the base coefficient b and every residual coefficient g_k (k <= j)
//    by d_j = m_j / sqrt(||V_j row||^2), with ||V_j row||^2 = b^2 nsq0 + sum_{k<=j} 2 s_k g_k b T2_k
//    + sum_{k,l<=j} s_k s_l g_k g_l G_kl, nsq0 = sum_in W^2 + in 1e-12, T2_k = rowsum((W A_k^T) * B_k),
//    G_kl = rowsum(B_k * (B_l A_l A_k^T)); then c0 = b and B'_k = g_k (.) B_k.
// The fold is pinned against the merge (tests/host/chain_test.cpp, the reference's own
// tests/lora_compose_test.cpp cases and inputs); the merge for one dora-rows adapter equals the
// materialised W_eff of the training oracle (orc_effective_weight, pinned in round trips of
// tests/test_oracle_dit_lin.py).
#include "oracle.h"

#include <cmath>
#include <vector>

namespace {

using dvec = std::vector<double>;

double scale_of(const orc_chain_adapter& a) { return (double)(a.alpha / (float)a.rank * a.strength); }

}  // namespace

extern "C" {

void orc_chain_merge(const float* W, int64_t in, int64_t out, int n, const orc_chain_adapter* ad, float* Weff) {
    dvec w((size_t)(in * out));
    for (int64_t k = 0; k < in * out; ++k) w[(size_t)k] = W[k];
    dvec v(w.size());
    for (int a = 0; a < n; ++a) {
        const orc_chain_adapter& x = ad[a];
        if (x.strength == 0.0f) continue;
        const double s = scale_of(x);
        for (int64_t o = 0; o < out; ++o) {
            for (int64_t i = 0; i < in; ++i) {
                double d = 0.0;
                for (int r = 0; r < x.rank; ++r) d += (double)x.B[o * x.rank + r] * x.A[r * in + i];
                v[(size_t)(o * in + i)] = w[(size_t)(o * in + i)] + s * d;
            }
            if (x.dora) {
                double ss = 0.0;
                for (int64_t i = 0; i < in; ++i) ss += v[(size_t)(o * in + i)] * v[(size_t)(o * in + i)];
                const double f = (double)x.mag[o] / std::sqrt(ss + (double)in * 1e-12);
                for (int64_t i = 0; i < in; ++i) v[(size_t)(o * in + i)] *= f;
            }
        }
        w.swap(v);
    }
    for (size_t k = 0; k < w.size(); ++k) Weff[k] = (float)w[k];
}

void orc_chain_fold(const float* W, int64_t in, int64_t out, int n, const orc_chain_adapter* ad, float* base_scale,
                    float* Bp, float* scales) {
    // the active adapters (strength != 0), in chain order
    std::vector<int> act;
    int R = 0;
    for (int a = 0; a < n; ++a)
        if (ad[a].strength != 0.0f) act.push_back(a);
    for (int a : act) R += ad[a].rank;
    const int M = (int)act.size();
    // grams A_l A_k^T per (k, l), [r_k][r_l]
    std::vector<dvec> gram((size_t)(M * M));
    for (int k = 0; k < M; ++k)
        for (int l = 0; l < M; ++l) {
            const orc_chain_adapter &ak = ad[act[k]], &al = ad[act[l]];
            dvec& g = gram[(size_t)(k * M + l)];
            g.assign((size_t)(ak.rank * al.rank), 0.0);
            for (int j = 0; j < ak.rank; ++j)
                for (int i = 0; i < al.rank; ++i) {
                    double s = 0.0;
                    for (int64_t c = 0; c < in; ++c) s += (double)ak.A[j * in + c] * al.A[i * in + c];
                    g[(size_t)(j * al.rank + i)] = s;
                }
        }
    for (int64_t o = 0; o < out; ++o) {
        const float* wo = W + o * in;
        double nsq0 = 0.0;
        for (int64_t c = 0; c < in; ++c) nsq0 += (double)wo[c] * wo[c];
        nsq0 += (double)in * 1e-12;
        dvec T2((size_t)M, 0.0), G((size_t)(M * M), 0.0), s((size_t)M), g((size_t)M, 1.0);
        for (int k = 0; k < M; ++k) {
            const orc_chain_adapter& ak = ad[act[k]];
            s[(size_t)k] = scale_of(ak);
            for (int j = 0; j < ak.rank; ++j) {
                double p = 0.0;
                for (int64_t c = 0; c < in; ++c) p += (double)wo[c] * ak.A[j * in + c];
                T2[(size_t)k] += p * ak.B[o * ak.rank + j];
            }
        }
        for (int k = 0; k < M; ++k)
            for (int l = 0; l < M; ++l) {
                const orc_chain_adapter &ak = ad[act[k]], &al = ad[act[l]];
                const dvec& gr = gram[(size_t)(k * M + l)];
                double acc = 0.0;
                for (int j = 0; j < ak.rank; ++j) {
                    double gb = 0.0;
                    for (int i = 0; i < al.rank; ++i) gb += gr[(size_t)(j * al.rank + i)] * al.B[o * al.rank + i];
                    acc += (double)ak.B[o * ak.rank + j] * gb;
                }
                G[(size_t)(k * M + l)] = acc;
            }
        double b = 1.0;
        for (int j = 0; j < M; ++j) {
            const orc_chain_adapter& aj = ad[act[j]];
            if (!aj.dora) continue;
            double nsq = b * b * nsq0;
            for (int k = 0; k <= j; ++k) nsq += 2.0 * s[(size_t)k] * g[(size_t)k] * b * T2[(size_t)k];
            for (int k = 0; k <= j; ++k)
                for (int l = 0; l <= j; ++l)
                    nsq += s[(size_t)k] * s[(size_t)l] * g[(size_t)k] * g[(size_t)l] * G[(size_t)(k * M + l)];
            const double d = (double)aj.mag[o] / std::sqrt(nsq);
            b *= d;
            for (int k = 0; k <= j; ++k) g[(size_t)k] *= d;
        }
        base_scale[o] = (float)b;
        int col = 0;
        for (int k = 0; k < M; ++k) {
            const orc_chain_adapter& ak = ad[act[k]];
            for (int j = 0; j < ak.rank; ++j) Bp[o * R + col + j] = (float)(g[(size_t)k] * ak.B[o * ak.rank + j]);
            col += ak.rank;
        }
    }
    for (int k = 0; k < M; ++k) scales[k] = (float)scale_of(ad[act[k]]);
}

void orc_chain_forward(const float* X, int64_t N, const float* W, int64_t in, int64_t out, int n,
                       const orc_chain_adapter* ad, const float* bias, float* Y) {
    int R = 0, M = 0;
    for (int a = 0; a < n; ++a)
        if (ad[a].strength != 0.0f) {
            R += ad[a].rank;
            ++M;
        }
    std::vector<float> c0((size_t)out), Bp((size_t)(out * (R > 0 ? R : 1))), sc((size_t)(M > 0 ? M : 1));
    orc_chain_fold(W, in, out, n, ad, c0.data(), Bp.data(), sc.data());
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < N; ++t) {
        const float* x = X + t * in;
        dvec h((size_t)(R > 0 ? R : 1));
        int col = 0, k = 0;
        for (int a = 0; a < n; ++a) {
            const orc_chain_adapter& aa = ad[a];
            if (aa.strength == 0.0f) continue;
            for (int j = 0; j < aa.rank; ++j) {
                double s = 0.0;
                for (int64_t c = 0; c < in; ++c) s += (double)x[c] * aa.A[j * in + c];
                h[(size_t)(col + j)] = (double)sc[(size_t)k] * s;
            }
            col += aa.rank;
            ++k;
        }
        for (int64_t o = 0; o < out; ++o) {
            double base = 0.0;
            for (int64_t c = 0; c < in; ++c) base += (double)W[o * in + c] * x[c];
            double y = (double)c0[(size_t)o] * base;
            for (int j = 0; j < R; ++j) y += h[(size_t)j] * Bp[(size_t)(o * R + j)];
            if (bias) y += bias[o];
            Y[t * out + o] = (float)y;
        }
    }
}

}  // extern "C"
