// oracle: the float kernels of the oracle's f32 mode (the CPU baseline) — TEST INFRASTRUCTURE ONLY.
//
// Built on its own with -O3 -mavx2 -mfma -ffp-contract=fast (x86-64-v3: every x86 host that
// carries an MI355X has it); the callers check the CPU first (orc_f32_kernels_ok, dit_lin.cpp) and
// use the generic loops otherwise. This file has no static initialisers, so nothing in it runs
// before that check.
//   orc_sgemm_nt  C = A . B^T, B packed into 16-column panels (k-major), 6 x 16 register tiles,
//                 OpenMP over (96-row block, panel) pairs
//   orc_sdot      float dot product (8 lanes, two accumulators)
//   orc_saxpy     y += a x
#include "oracle_f32.h"

#include <cstddef>
#include <vector>

namespace {

typedef float v8 __attribute__((vector_size(32)));

constexpr int MR = 6, NR = 16;
constexpr int64_t MC = 96;

inline v8 ld(const float* p) {
    v8 v;
    __builtin_memcpy(&v, p, sizeof(v));
    return v;
}
inline void st(float* p, v8 v) { __builtin_memcpy(p, &v, sizeof(v)); }
inline v8 bc(float a) { return v8{a, a, a, a, a, a, a, a}; }

// C[m0 + i][n0 + j] for i < mr, j < nr, over the full K: rows past mr read row 0 of the group
void micro(const float* const* arow, const float* bp, int64_t K, float* C, int64_t ldc, int mr, int nr) {
    v8 c[MR][2];
    for (int i = 0; i < MR; ++i) c[i][0] = c[i][1] = bc(0.f);
    for (int64_t k = 0; k < K; ++k) {
        const v8 b0 = ld(bp + k * NR), b1 = ld(bp + k * NR + 8);
#pragma GCC unroll 6
        for (int i = 0; i < MR; ++i) {
            const v8 a = bc(arow[i][k]);
            c[i][0] += a * b0;
            c[i][1] += a * b1;
        }
    }
    for (int i = 0; i < mr; ++i) {
        float* crow = C + i * ldc;
        if (nr == NR) {
            st(crow, c[i][0]);
            st(crow + 8, c[i][1]);
        } else {
            float t[NR];
            st(t, c[i][0]);
            st(t + 8, c[i][1]);
            for (int j = 0; j < nr; ++j) crow[j] = t[j];
        }
    }
}

}  // namespace

void orc_sgemm_nt(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0) return;
    const int64_t NP = (N + NR - 1) / NR;
    std::vector<float> Bp((std::size_t)(NP * K * NR));
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < NP; ++p) {
        float* d = Bp.data() + (std::size_t)(p * K * NR);
        for (int j = 0; j < NR; ++j) {
            const int64_t n = p * NR + j;
            if (n < N) {
                const float* s = B + n * K;
                for (int64_t k = 0; k < K; ++k) d[k * NR + j] = s[k];
            } else {
                for (int64_t k = 0; k < K; ++k) d[k * NR + j] = 0.f;
            }
        }
    }
    const int64_t MB = (M + MC - 1) / MC;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t mb = 0; mb < MB; ++mb)
        for (int64_t p = 0; p < NP; ++p) {
            const int64_t n0 = p * NR;
            const int nr = (int)(N - n0 < NR ? N - n0 : NR);
            const int64_t m_end = (mb + 1) * MC < M ? (mb + 1) * MC : M;
            for (int64_t m0 = mb * MC; m0 < m_end; m0 += MR) {
                const int mr = (int)(m_end - m0 < MR ? m_end - m0 : MR);
                const float* arow[MR];
                for (int i = 0; i < MR; ++i) arow[i] = A + (m0 + (i < mr ? i : 0)) * K;
                micro(arow, Bp.data() + (std::size_t)(p * K * NR), K, C + m0 * N + n0, N, mr, nr);
            }
        }
}

float orc_sdot(const float* a, const float* b, int n) {
    v8 s0 = bc(0.f), s1 = bc(0.f);
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        s0 += ld(a + i) * ld(b + i);
        s1 += ld(a + i + 8) * ld(b + i + 8);
    }
    for (; i + 8 <= n; i += 8) s0 += ld(a + i) * ld(b + i);
    s0 += s1;
    float s = ((s0[0] + s0[4]) + (s0[1] + s0[5])) + ((s0[2] + s0[6]) + (s0[3] + s0[7]));
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

void orc_saxpy(float a, const float* x, float* y, int n) {
    const v8 av = bc(a);
    int i = 0;
    for (; i + 8 <= n; i += 8) st(y + i, ld(y + i) + av * ld(x + i));
    for (; i < n; ++i) y[i] += a * x[i];
}
