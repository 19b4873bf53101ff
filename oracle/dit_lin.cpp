// oracle: adapter state and the functional LoRA/DoRA linear — TEST INFRASTRUCTURE ONLY.
//
// dit_lin (src/dit.h:92-149) is a ggml graph in the reference; here its forward is restated op by
// op in double precision, and its backward is the closed form of the ggml autodiff result:
//   gd = sum_n dY*U, dm = gd/sqrt(nsq), gn = -1/2 gd m nsq^-3/2, dU = dY*d,
//   dX = dU W + s (dU B) A,
//   dB = s dU^T H + 2s diag(gn) P + 2s^2 diag(gn) B G,
//   dA = s (dU B)^T X + 2s B^T diag(gn) W + 2s^2 (B^T diag(gn) B) A,
// with H = X A^T, P = W A^T, G = A A^T (lora: d = 1, gn = 0). The closed form is pinned by
// central finite differences of the double forward and by torch autograd fixtures (tests/).
#include "oracle.h"
#include "oracle_f32.h"

#include <malloc.h>

#include <cmath>
#include <cstring>
#include <type_traits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

int g_orc_f32 = 0;

bool orc_f32_kernels_ok() { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }

namespace {

// R: the compute type, double (the oracle) or float (orc_set_f32: the CPU baseline)
template <class R>
using rvec = std::vector<R>;
using dvec = rvec<double>;

template <class R>
rvec<R> to_r(const float* x, int64_t n) {
    return rvec<R>(x, x + n);
}

// C[M][N] = sum_k A[M][K] * B[N][K]  (both K-contiguous)
template <class R>
void mm_nt(const R* A, const R* B, R* C, int64_t M, int64_t N, int64_t K) {
    if constexpr (std::is_same<R, float>::value) {
        if (orc_f32_kernels_ok()) {
            orc_sgemm_nt(A, B, C, M, N, K);
            return;
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const R* a = A + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const R* b = B + n * K;
            R s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            int64_t k = 0;
            for (; k + 4 <= K; k += 4) {
                s0 += a[k] * b[k];
                s1 += a[k + 1] * b[k + 1];
                s2 += a[k + 2] * b[k + 2];
                s3 += a[k + 3] * b[k + 3];
            }
            for (; k < K; ++k) s0 += a[k] * b[k];
            C[m * N + n] = (s0 + s1) + (s2 + s3);
        }
    }
}

template <class R>
rvec<R> transpose(const R* A, int64_t Rn, int64_t Cn) {
    rvec<R> t((size_t)(Rn * Cn));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < Rn; ++r)
        for (int64_t c = 0; c < Cn; ++c) t[(size_t)(c * Rn + r)] = A[r * Cn + c];
    return t;
}

template <class R>
struct DoraTerms {
    rvec<R> P, G, nsq, d;  // P [out][r], G [r][r], nsq/d [out]
};

template <class R>
DoraTerms<R> dora_terms(const rvec<R>& W, const rvec<R>& A, const rvec<R>& B, int64_t in, int64_t out, int r,
                        R s, int dora, const float* mag, const float* bnsq) {
    DoraTerms<R> t;
    t.d.assign((size_t)out, 1);
    t.nsq.assign((size_t)out, 1);
    if (!dora) return t;
    t.P.resize((size_t)(out * r));
    mm_nt(W.data(), A.data(), t.P.data(), out, r, in);            // W A^T
    t.G.resize((size_t)(r * r));
    mm_nt(A.data(), A.data(), t.G.data(), r, r, in);              // A A^T
    for (int64_t o = 0; o < out; ++o) {
        R t2 = 0, t3 = 0;
        for (int a = 0; a < r; ++a) {
            t2 += t.P[(size_t)(o * r + a)] * B[(size_t)(o * r + a)];
            R gb = 0;
            for (int b = 0; b < r; ++b) gb += t.G[(size_t)(a * r + b)] * B[(size_t)(o * r + b)];
            t3 += B[(size_t)(o * r + a)] * gb;
        }
        const R nsq = (R)bnsq[o] + 2 * s * t2 + s * s * t3;
        t.nsq[(size_t)o] = nsq;
        t.d[(size_t)o] = (R)mag[o] / std::sqrt(nsq);
    }
    return t;
}

// src/dit.h:92-149: y = W x (+ s B A x), dora: y *= m / sqrt(bnsq + 2s t2 + s^2 t3), then + bias
template <class R>
void dit_lin_fwd_impl(const float* Xf, int64_t N, const float* Wf, int64_t in, int64_t out, const float* Af,
                      const float* Bf, int r, float sf, int dora, const float* mag, const float* bnsq,
                      const float* bias, float* Y, float* U, float* dscale, float* nsq_out,
                      std::vector<double>* Yd) {
    const R s = sf;
    rvec<R> X = to_r<R>(Xf, N * in), W = to_r<R>(Wf, out * in);
    rvec<R> A = r ? to_r<R>(Af, (int64_t)r * in) : rvec<R>(), B = r ? to_r<R>(Bf, out * r) : rvec<R>();
    rvec<R> Y0((size_t)(N * out));
    mm_nt(X.data(), W.data(), Y0.data(), N, out, in);
    if (r > 0) {
        rvec<R> H((size_t)(N * r));
        mm_nt(X.data(), A.data(), H.data(), N, r, in);
        rvec<R> BAX((size_t)(N * out));
        mm_nt(H.data(), B.data(), BAX.data(), N, out, r);   // (X A^T) B^T: B [out][r] is K-contiguous
        for (size_t i = 0; i < Y0.size(); ++i) Y0[i] += s * BAX[i];
    }
    DoraTerms<R> t = dora_terms<R>(W, A, B, in, out, r, s, dora && r > 0, mag, bnsq);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t o = 0; o < out; ++o) {
            const R u = Y0[(size_t)(n * out + o)];
            if (U) U[n * out + o] = (float)u;
            R y = u * t.d[(size_t)o];
            if (bias) y += bias[o];
            if (Y) Y[n * out + o] = (float)y;
            if (Yd) (*Yd)[(size_t)(n * out + o)] = (double)y;
        }
    if (dscale)
        for (int64_t o = 0; o < out; ++o) dscale[o] = (float)t.d[(size_t)o];
    if (nsq_out)
        for (int64_t o = 0; o < out; ++o) nsq_out[o] = (float)t.nsq[(size_t)o];
}

template <class R>
void dit_lin_bwd_impl(const float* Xf, int64_t N, const float* Wf, int64_t in, int64_t out, const float* Af,
                      const float* Bf, int r, float sf, int dora, const float* mag, const float* bnsq,
                      const float* dYf, float* dX, float* dA, float* dB, float* dm) {
    const R s = sf;
    rvec<R> X = to_r<R>(Xf, N * in), W = to_r<R>(Wf, out * in), dY = to_r<R>(dYf, N * out);
    rvec<R> A = r ? to_r<R>(Af, (int64_t)r * in) : rvec<R>(), B = r ? to_r<R>(Bf, out * r) : rvec<R>();
    const bool isdora = dora && r > 0;
    DoraTerms<R> t = dora_terms<R>(W, A, B, in, out, r, s, isdora, mag, bnsq);
    rvec<R> H;
    if (r > 0) {
        H.resize((size_t)(N * r));
        mm_nt(X.data(), A.data(), H.data(), N, r, in);
    }
    // gd needs U = X W^T + s H B^T
    rvec<R> gn((size_t)out, 0.0);
    if (isdora) {
        rvec<R> U((size_t)(N * out));
        mm_nt(X.data(), W.data(), U.data(), N, out, in);
        rvec<R> BAX((size_t)(N * out));
        mm_nt(H.data(), B.data(), BAX.data(), N, out, r);   // (X A^T) B^T: B [out][r] is K-contiguous
        rvec<R> gd((size_t)out, 0.0);
        for (int64_t n = 0; n < N; ++n)
            for (int64_t o = 0; o < out; ++o) {
                const size_t k = (size_t)(n * out + o);
                gd[(size_t)o] += dY[k] * (U[k] + s * BAX[k]);
            }
        for (int64_t o = 0; o < out; ++o) {
            const R nsq = t.nsq[(size_t)o];
            if (dm) dm[o] = (float)(gd[(size_t)o] / std::sqrt(nsq));
            gn[(size_t)o] = -(R)0.5 * gd[(size_t)o] * (R)mag[o] / (nsq * std::sqrt(nsq));
        }
    } else if (dm) {
        for (int64_t o = 0; o < out; ++o) dm[o] = 0.0f;
    }
    // dU = dY * d
    rvec<R> dU((size_t)(N * out));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t o = 0; o < out; ++o) dU[(size_t)(n * out + o)] = dY[(size_t)(n * out + o)] * t.d[(size_t)o];
    rvec<R> dUt = transpose(dU.data(), N, out);  // [out][N]
    if (dX) {
        rvec<R> Wt = transpose(W.data(), out, in);  // [in][out]
        rvec<R> dXd((size_t)(N * in));
        mm_nt(dU.data(), Wt.data(), dXd.data(), N, in, out);
        if (r > 0) {
            rvec<R> dUB((size_t)(N * r));
            mm_nt(dU.data(), transpose(B.data(), out, r).data(), dUB.data(), N, r, out);
            rvec<R> At = transpose(A.data(), r, in);  // [in][r]
            rvec<R> t2((size_t)(N * in));
            mm_nt(dUB.data(), At.data(), t2.data(), N, in, r);
            for (size_t i = 0; i < dXd.size(); ++i) dXd[i] += s * t2[i];
        }
        for (int64_t i = 0; i < N * in; ++i) dX[i] = (float)dXd[(size_t)i];
    }
    if (r == 0) return;
    if (dB) {
        rvec<R> Ht = transpose(H.data(), N, r);  // [r][N]
        rvec<R> dBd((size_t)(out * r));
        mm_nt(dUt.data(), Ht.data(), dBd.data(), out, r, N);
        for (int64_t o = 0; o < out; ++o)
            for (int a = 0; a < r; ++a) {
                R v = s * dBd[(size_t)(o * r + a)];
                if (isdora) {
                    R bg = 0;
                    for (int b = 0; b < r; ++b) bg += B[(size_t)(o * r + b)] * t.G[(size_t)(b * r + a)];
                    v += 2 * s * gn[(size_t)o] * t.P[(size_t)(o * r + a)] + 2 * s * s * gn[(size_t)o] * bg;
                }
                dB[o * r + a] = (float)v;
            }
    }
    if (dA) {
        rvec<R> dUB((size_t)(N * r));
        mm_nt(dU.data(), transpose(B.data(), out, r).data(), dUB.data(), N, r, out);
        rvec<R> dUBt = transpose(dUB.data(), N, r);      // [r][N]
        rvec<R> Xt = transpose(X.data(), N, in);         // [in][N]
        rvec<R> dAd((size_t)(r * in));
        mm_nt(dUBt.data(), Xt.data(), dAd.data(), r, in, N);
        for (auto& v : dAd) v *= s;
        if (isdora) {
            // 2s B^T diag(gn) W  and  2s^2 (B^T diag(gn) B) A
            rvec<R> Bg((size_t)(r * out));  // [r][out] = B^T diag(gn)
            for (int64_t o = 0; o < out; ++o)
                for (int a = 0; a < r; ++a) Bg[(size_t)(a * out + o)] = B[(size_t)(o * r + a)] * gn[(size_t)o];
            rvec<R> Wt = transpose(W.data(), out, in);      // [in][out]
            rvec<R> T1((size_t)(r * in));
            mm_nt(Bg.data(), Wt.data(), T1.data(), r, in, out);
            rvec<R> BgB((size_t)(r * r));                   // [r][r] = B^T diag(gn) B
            rvec<R> Bt = transpose(B.data(), out, r);       // [r][out]
            mm_nt(Bg.data(), Bt.data(), BgB.data(), r, r, out);
            rvec<R> At = transpose(A.data(), r, in);        // [in][r]
            rvec<R> T2((size_t)(r * in));
            mm_nt(BgB.data(), At.data(), T2.data(), r, in, r);
            for (size_t i = 0; i < dAd.size(); ++i) dAd[i] += 2 * s * T1[i] + 2 * s * s * T2[i];
        }
        for (int64_t i = 0; i < (int64_t)r * in; ++i) dA[i] = (float)dAd[(size_t)i];
    }
}

}  // namespace

extern "C" {

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// src/train_lora.h:160-174 (f32 data, double sum, + in*eps)
void orc_row_norm_sq(const float* W, int64_t in, int64_t out, float eps, float* nsq) {
    for (int64_t o = 0; o < out; ++o) {
        double s = 0.0;
        for (int64_t i = 0; i < in; ++i) {
            const float v = W[o * in + i];
            s += (double)v * v;
        }
        nsq[o] = (float)(s + (double)in * eps);
    }
}

// src/train_lora.h:141-155
void orc_row_norms(const float* W, int64_t in, int64_t out, float* norms) {
    for (int64_t o = 0; o < out; ++o) {
        double s = 0.0;
        for (int64_t i = 0; i < in; ++i) {
            const float v = W[o * in + i];
            s += (double)v * v;
        }
        norms[o] = (float)std::sqrt(s);
    }
}

// src/train_lora.h:301-329 for "lora" and "dora-rows": v = W + (alpha/r) B A;
// dora-rows: v_o * mag_o / sqrt(sum_i v_oi^2 + in*1e-12) (rms_norm(v, 1e-12) / sqrt(in) * mag)
void orc_effective_weight(const float* W, int64_t in, int64_t out, const float* A, const float* B,
                          const float* mag, int rank, float alpha, int dora, float* Weff) {
    const double s = (double)alpha / (double)rank;
    for (int64_t o = 0; o < out; ++o) {
        std::vector<double> row((size_t)in);
        double ss = 0.0;
        for (int64_t i = 0; i < in; ++i) {
            double d = 0.0;
            for (int a = 0; a < rank; ++a) d += (double)B[o * rank + a] * A[a * in + i];
            row[(size_t)i] = (double)W[o * in + i] + s * d;
            ss += row[(size_t)i] * row[(size_t)i];
        }
        const double sc = dora ? (double)mag[o] / std::sqrt(ss + (double)in * 1e-12) : 1.0;
        for (int64_t i = 0; i < in; ++i) Weff[o * in + i] = (float)(row[(size_t)i] * sc);
    }
}

void orc_gemm_nt(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
    dvec a = to_r<double>(A, M * K), b = to_r<double>(B, N * K), c((size_t)(M * N));
    mm_nt(a.data(), b.data(), c.data(), M, N, K);
    for (int64_t i = 0; i < M * N; ++i) C[i] = (float)c[(size_t)i];
}

void orc_dit_lin_fwd(const float* Xf, int64_t N, const float* Wf, int64_t in, int64_t out,
                     const float* Af, const float* Bf, int r, float sf, int dora, const float* mag,
                     const float* bnsq, const float* bias, float* Y, float* U, float* dscale,
                     float* nsq_out) {
    if (g_orc_f32)
        dit_lin_fwd_impl<float>(Xf, N, Wf, in, out, Af, Bf, r, sf, dora, mag, bnsq, bias, Y, U, dscale, nsq_out, nullptr);
    else
        dit_lin_fwd_impl<double>(Xf, N, Wf, in, out, Af, Bf, r, sf, dora, mag, bnsq, bias, Y, U, dscale, nsq_out, nullptr);
}

// sum (Y - tgt)^2 with Y kept in double (for finite-difference checks of the backward)
double orc_dit_lin_sqloss(const float* Xf, int64_t N, const float* Wf, int64_t in, int64_t out,
                          const float* Af, const float* Bf, int r, float sf, int dora, const float* mag,
                          const float* bnsq, const float* bias, const float* tgt) {
    std::vector<double> Yd((size_t)(N * out));
    dit_lin_fwd_impl<double>(Xf, N, Wf, in, out, Af, Bf, r, sf, dora, mag, bnsq, bias, nullptr, nullptr, nullptr,
                             nullptr, &Yd);
    double l = 0.0;
    for (size_t i = 0; i < Yd.size(); ++i) l += (Yd[i] - tgt[i]) * (Yd[i] - tgt[i]);
    return l;
}

void orc_dit_lin_bwd(const float* Xf, int64_t N, const float* Wf, int64_t in, int64_t out,
                     const float* Af, const float* Bf, int r, float sf, int dora, const float* mag,
                     const float* bnsq, const float* dYf, float* dX, float* dA, float* dB, float* dm) {
    if (g_orc_f32)
        dit_lin_bwd_impl<float>(Xf, N, Wf, in, out, Af, Bf, r, sf, dora, mag, bnsq, dYf, dX, dA, dB, dm);
    else
        dit_lin_bwd_impl<double>(Xf, N, Wf, in, out, Af, Bf, r, sf, dora, mag, bnsq, dYf, dX, dA, dB, dm);
}

// The f32 mode is the timed CPU baseline. Its loops allocate and free GB-sized temporaries, which
// glibc otherwise maps fresh from the kernel each time (page faults and zeroing in the timed
// region). Switching the mode on keeps freed memory in the process heap for reuse.
void orc_set_f32(int on) {
    if (on) {
        mallopt(M_MMAP_MAX, 0);
        mallopt(M_TRIM_THRESHOLD, 1 << 30);
        mallopt(M_TOP_PAD, 64 << 20);
    }
    g_orc_f32 = on ? 1 : 0;
}
int orc_f32_fast(void) { return orc_f32_kernels_ok() ? 1 : 0; }

}  // extern "C"
