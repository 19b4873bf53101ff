// oracle: differential attention forward and backward — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// The DiT's attention (src/dit.h:151-158 dit_diff_attn over nn::sdpa, src/nn.h:135-144): per
// (batch, head), two softmax attentions that share V and are subtracted,
//   O = softmax(Q1 K1^T * scale) V - softmax(Q2 K2^T * scale) V,
// dense (no mask) in the reference; window > 0 restricts query i to keys j with |i - j| <= window/2
// (the banded variant the sliding-window configuration asks for; window 0 is the reference).
// Backward is the textbook softmax-attention gradient per branch with dO_2 = -dO:
//   dP = dO_i V^T, dS = P (dP - rowsum(P dP)), dQ = scale dS K, dK = scale dS^T Q, dV += P^T dO_i.
// Double accumulation throughout; pinned by central finite differences and torch autograd fixtures.
#include "oracle.h"

#include <cmath>
#include <vector>

namespace {

inline bool visible(int i, int j, int window) {
    if (window <= 0) return true;
    const int d = i > j ? i - j : j - i;
    return 2 * d <= window;
}

// P [Sq][Sk] = softmax(scale Q K^T) (masked entries 0); lse [Sq]
void probs(const float* Q, const float* K, int Sq, int Sk, int D, double scale, int window,
           std::vector<double>& P, std::vector<double>& lse) {
    P.assign((size_t)Sq * Sk, 0.0);
    lse.assign((size_t)Sq, 0.0);
    for (int i = 0; i < Sq; ++i) {
        double m = -INFINITY;
        for (int j = 0; j < Sk; ++j) {
            if (!visible(i, j, window)) continue;
            double s = 0.0;
            for (int d = 0; d < D; ++d) s += (double)Q[(size_t)i * D + d] * K[(size_t)j * D + d];
            s *= scale;
            P[(size_t)i * Sk + j] = s;
            if (s > m) m = s;
        }
        double l = 0.0;
        for (int j = 0; j < Sk; ++j) {
            if (!visible(i, j, window)) continue;
            const double e = std::exp(P[(size_t)i * Sk + j] - m);
            P[(size_t)i * Sk + j] = e;
            l += e;
        }
        for (int j = 0; j < Sk; ++j) P[(size_t)i * Sk + j] /= l;
        lse[(size_t)i] = m + std::log(l);
    }
}

}  // namespace

extern "C" {

void orc_diff_attn_fwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       int BH, int Sq, int Sk, int D, float scale, int window, float* O, float* O1, float* O2,
                       float* lse1, float* lse2) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < BH; ++bh) {
        const size_t qo = (size_t)bh * Sq * D, ko = (size_t)bh * Sk * D;
        std::vector<double> P1, P2, l1, l2;
        probs(Q1 + qo, K1 + ko, Sq, Sk, D, scale, window, P1, l1);
        probs(Q2 + qo, K2 + ko, Sq, Sk, D, scale, window, P2, l2);
        for (int i = 0; i < Sq; ++i) {
            for (int d = 0; d < D; ++d) {
                double a = 0.0, b = 0.0;
                for (int j = 0; j < Sk; ++j) {
                    const double v = V[ko + (size_t)j * D + d];
                    a += P1[(size_t)i * Sk + j] * v;
                    b += P2[(size_t)i * Sk + j] * v;
                }
                O[qo + (size_t)i * D + d] = (float)(a - b);
                if (O1) O1[qo + (size_t)i * D + d] = (float)a;
                if (O2) O2[qo + (size_t)i * D + d] = (float)b;
            }
            if (lse1) lse1[(size_t)bh * Sq + i] = (float)l1[(size_t)i];
            if (lse2) lse2[(size_t)bh * Sq + i] = (float)l2[(size_t)i];
        }
    }
}

void orc_diff_attn_bwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       const float* dO, int BH, int Sq, int Sk, int D, float scale, int window, float* dQ1,
                       float* dK1, float* dQ2, float* dK2, float* dV) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < BH; ++bh) {
        const size_t qo = (size_t)bh * Sq * D, ko = (size_t)bh * Sk * D;
        std::vector<double> dv((size_t)Sk * D, 0.0);
        for (int br = 0; br < 2; ++br) {
            const float* Q = br == 0 ? Q1 : Q2;
            const float* K = br == 0 ? K1 : K2;
            float* dQ = br == 0 ? dQ1 : dQ2;
            float* dK = br == 0 ? dK1 : dK2;
            const double sign = br == 0 ? 1.0 : -1.0;
            std::vector<double> P, lse;
            probs(Q + qo, K + ko, Sq, Sk, D, scale, window, P, lse);
            std::vector<double> dS((size_t)Sq * Sk, 0.0);
            for (int i = 0; i < Sq; ++i) {
                double rs = 0.0;
                for (int j = 0; j < Sk; ++j) {
                    double dp = 0.0;
                    for (int d = 0; d < D; ++d) dp += (double)dO[qo + (size_t)i * D + d] * V[ko + (size_t)j * D + d];
                    dp *= sign;
                    dS[(size_t)i * Sk + j] = dp;
                    rs += P[(size_t)i * Sk + j] * dp;
                }
                for (int j = 0; j < Sk; ++j)
                    dS[(size_t)i * Sk + j] = P[(size_t)i * Sk + j] * (dS[(size_t)i * Sk + j] - rs);
            }
            for (int i = 0; i < Sq; ++i)
                for (int d = 0; d < D; ++d) {
                    double a = 0.0;
                    for (int j = 0; j < Sk; ++j) a += dS[(size_t)i * Sk + j] * K[ko + (size_t)j * D + d];
                    dQ[qo + (size_t)i * D + d] = (float)(scale * a);
                }
            for (int j = 0; j < Sk; ++j)
                for (int d = 0; d < D; ++d) {
                    double a = 0.0, b = 0.0;
                    for (int i = 0; i < Sq; ++i) {
                        a += dS[(size_t)i * Sk + j] * Q[qo + (size_t)i * D + d];
                        b += P[(size_t)i * Sk + j] * dO[qo + (size_t)i * D + d];
                    }
                    dK[ko + (size_t)j * D + d] = (float)(scale * a);
                    dv[(size_t)j * D + d] += sign * b;
                }
        }
        for (size_t k = 0; k < dv.size(); ++k) dV[ko + k] = (float)dv[k];
    }
}

}  // extern "C"
