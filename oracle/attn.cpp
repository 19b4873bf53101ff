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
// Every sum runs over the visible keys (or queries) only, in increasing index order: the masked
// terms are exact zeros, so skipping them leaves each sum as it was. In the f32 mode (orc_set_f32,
// the CPU baseline) the same loops run in float with sgemm.cpp's dot and axpy kernels.
#include "oracle.h"
#include "oracle_f32.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

namespace {

// keys j visible from query i: |i - j| <= window / 2 (window 0: all)
inline void key_range(int i, int Sk, int window, int& lo, int& hi) {
    if (window <= 0) {
        lo = 0;
        hi = Sk - 1;
        return;
    }
    const int h = window / 2;
    lo = std::max(0, i - h);
    hi = std::min(Sk - 1, i + h);
}

template <class R>
inline R dot(const float* a, const float* b, int n) {
    if constexpr (std::is_same<R, float>::value) {
        if (orc_f32_kernels_ok()) return orc_sdot(a, b, n);
    }
    R s = 0;
    for (int d = 0; d < n; ++d) s += (R)a[d] * b[d];
    return s;
}

// y[0..n) += a * x (x float)
template <class R>
inline void axpy(R a, const float* x, R* y, int n) {
    if constexpr (std::is_same<R, float>::value) {
        if (orc_f32_kernels_ok()) {
            orc_saxpy(a, x, y, n);
            return;
        }
    }
    for (int d = 0; d < n; ++d) y[d] += a * x[d];
}

// P [Sq][Sk] = softmax(scale Q K^T) (masked entries 0); lse [Sq]
template <class R>
void probs(const float* Q, const float* K, int Sq, int Sk, int D, R scale, int window, std::vector<R>& P,
           std::vector<R>& lse) {
    P.assign((size_t)Sq * Sk, 0);
    lse.assign((size_t)Sq, 0);
    for (int i = 0; i < Sq; ++i) {
        int lo, hi;
        key_range(i, Sk, window, lo, hi);
        R* p = &P[(size_t)i * Sk];
        R m = -INFINITY;
        for (int j = lo; j <= hi; ++j) {
            const R s = dot<R>(Q + (size_t)i * D, K + (size_t)j * D, D) * scale;
            p[j] = s;
            if (s > m) m = s;
        }
        R l = 0;
        for (int j = lo; j <= hi; ++j) {
            const R e = std::exp(p[j] - m);
            p[j] = e;
            l += e;
        }
        for (int j = lo; j <= hi; ++j) p[j] /= l;
        lse[(size_t)i] = m + std::log(l);
    }
}

template <class R>
void fwd_impl(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V, int BH, int Sq,
              int Sk, int D, float scale, int window, float* O, float* O1, float* O2, float* lse1, float* lse2) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < BH; ++bh) {
        const size_t qo = (size_t)bh * Sq * D, ko = (size_t)bh * Sk * D;
        std::vector<R> P1, P2, l1, l2, a((size_t)D), b((size_t)D);
        probs<R>(Q1 + qo, K1 + ko, Sq, Sk, D, scale, window, P1, l1);
        probs<R>(Q2 + qo, K2 + ko, Sq, Sk, D, scale, window, P2, l2);
        for (int i = 0; i < Sq; ++i) {
            int lo, hi;
            key_range(i, Sk, window, lo, hi);
            std::fill(a.begin(), a.end(), (R)0);
            std::fill(b.begin(), b.end(), (R)0);
            for (int j = lo; j <= hi; ++j) {
                axpy<R>(P1[(size_t)i * Sk + j], V + ko + (size_t)j * D, a.data(), D);
                axpy<R>(P2[(size_t)i * Sk + j], V + ko + (size_t)j * D, b.data(), D);
            }
            for (int d = 0; d < D; ++d) {
                O[qo + (size_t)i * D + d] = (float)(a[(size_t)d] - b[(size_t)d]);
                if (O1) O1[qo + (size_t)i * D + d] = (float)a[(size_t)d];
                if (O2) O2[qo + (size_t)i * D + d] = (float)b[(size_t)d];
            }
            if (lse1) lse1[(size_t)bh * Sq + i] = (float)l1[(size_t)i];
            if (lse2) lse2[(size_t)bh * Sq + i] = (float)l2[(size_t)i];
        }
    }
}

template <class R>
void bwd_impl(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V, const float* dO,
              int BH, int Sq, int Sk, int D, float scale, int window, float* dQ1, float* dK1, float* dQ2, float* dK2,
              float* dV) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < BH; ++bh) {
        const size_t qo = (size_t)bh * Sq * D, ko = (size_t)bh * Sk * D;
        std::vector<R> dv((size_t)Sk * D, 0), acc((size_t)D), acc2((size_t)D);
        for (int br = 0; br < 2; ++br) {
            const float* Q = br == 0 ? Q1 : Q2;
            const float* K = br == 0 ? K1 : K2;
            float* dQ = br == 0 ? dQ1 : dQ2;
            float* dK = br == 0 ? dK1 : dK2;
            const R sign = br == 0 ? 1 : -1;
            std::vector<R> P, lse;
            probs<R>(Q + qo, K + ko, Sq, Sk, D, scale, window, P, lse);
            std::vector<R> dS((size_t)Sq * Sk, 0);
            for (int i = 0; i < Sq; ++i) {
                int lo, hi;
                key_range(i, Sk, window, lo, hi);
                R rs = 0;
                for (int j = lo; j <= hi; ++j) {
                    const R dp = dot<R>(dO + qo + (size_t)i * D, V + ko + (size_t)j * D, D) * sign;
                    dS[(size_t)i * Sk + j] = dp;
                    rs += P[(size_t)i * Sk + j] * dp;
                }
                for (int j = lo; j <= hi; ++j)
                    dS[(size_t)i * Sk + j] = P[(size_t)i * Sk + j] * (dS[(size_t)i * Sk + j] - rs);
            }
            // dQ_i = scale sum_j dS_ij K_j
            for (int i = 0; i < Sq; ++i) {
                int lo, hi;
                key_range(i, Sk, window, lo, hi);
                std::fill(acc.begin(), acc.end(), (R)0);
                for (int j = lo; j <= hi; ++j) axpy<R>(dS[(size_t)i * Sk + j], K + ko + (size_t)j * D, acc.data(), D);
                for (int d = 0; d < D; ++d) dQ[qo + (size_t)i * D + d] = (float)(scale * acc[(size_t)d]);
            }
            // dK_j = scale sum_i dS_ij Q_i, dV_j += sign sum_i P_ij dO_i (queries i that see key j)
            for (int j = 0; j < Sk; ++j) {
                int lo, hi;
                key_range(j, Sq, window, lo, hi);
                std::fill(acc.begin(), acc.end(), (R)0);
                std::fill(acc2.begin(), acc2.end(), (R)0);
                for (int i = lo; i <= hi; ++i) {
                    axpy<R>(dS[(size_t)i * Sk + j], Q + qo + (size_t)i * D, acc.data(), D);
                    axpy<R>(P[(size_t)i * Sk + j], dO + qo + (size_t)i * D, acc2.data(), D);
                }
                for (int d = 0; d < D; ++d) {
                    dK[ko + (size_t)j * D + d] = (float)(scale * acc[(size_t)d]);
                    dv[(size_t)j * D + d] += sign * acc2[(size_t)d];
                }
            }
        }
        for (size_t k = 0; k < dv.size(); ++k) dV[ko + k] = (float)dv[k];
    }
}

}  // namespace

extern "C" {

void orc_diff_attn_fwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       int BH, int Sq, int Sk, int D, float scale, int window, float* O, float* O1, float* O2,
                       float* lse1, float* lse2) {
    if (g_orc_f32) fwd_impl<float>(Q1, K1, Q2, K2, V, BH, Sq, Sk, D, scale, window, O, O1, O2, lse1, lse2);
    else fwd_impl<double>(Q1, K1, Q2, K2, V, BH, Sq, Sk, D, scale, window, O, O1, O2, lse1, lse2);
}

void orc_diff_attn_bwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       const float* dO, int BH, int Sq, int Sk, int D, float scale, int window, float* dQ1,
                       float* dK1, float* dQ2, float* dK2, float* dV) {
    if (g_orc_f32) bwd_impl<float>(Q1, K1, Q2, K2, V, dO, BH, Sq, Sk, D, scale, window, dQ1, dK1, dQ2, dK2, dV);
    else bwd_impl<double>(Q1, K1, Q2, K2, V, dO, BH, Sq, Sk, D, scale, window, dQ1, dK1, dQ2, dK2, dV);
}

}  // extern "C"
