// K1-K4: the functional LoRA / DoRA-rows linear of the DiT (dit_lin, src/dit.h:92-149), forward
// and backward, on top of the MFMA GEMM (gemm.h) and three small families of kernels:
//   * frozen weights:   layout once at load (forward [out][in] + transposed [in][out]; Q8_0 blocks
//                       split into int8 quants and f16 scales, bit-for-bit), row norms
//                       (train_row_norm_sq / train_row_norms, src/train_lora.h:141-174)
//   * adapter prepare:  once per optimizer step: P^T = A W^T (W-streaming GEMM), G = A A^T,
//                       t2, t3, nsq = bnsq + 2s t2 + s^2 t3, d = m / sqrt(nsq)  (src/dit.h:123-145)
//   * column reductions over the token axis (K3): gd = sum_n dY*U, dU^T H, (s dU B)^T X
//
// Forward (per call):   Hc = s X A^T                      (skinny GEMM)
//                       Y  = (X W^T + Hc B^T) * d + bias  (one GEMM: K-extension + epilogue)
// Backward (per call):  dU = dY*d, gd, dU^T Hc             (column reduction, writes dU)
//                       dm += gd/sqrt(nsq), gn = -gd m nsq^-3/2 / 2,
//                       dB += dU^T Hc + 2s gn P + 2s^2 gn B G
//                       sdUB = s dU B                      (skinny GEMM)
//                       dX = dU W + sdUB A  and, as r extra GEMM rows sharing the W^T tiles,
//                       dA += 2s B^T diag(gn) W + 2s^2 (B^T diag(gn) B) A
//                       dA += sdUB^T X                     (column reduction)
#include "lora.h"

#include <algorithm>
#include <cmath>
#include <set>
#include <string>
#include <vector>

using namespace sa3k;

struct sa3k_lin {
    const sa3k_weight* W = nullptr;
    int rank = 0, prec = SA3K_PREC_BF16, dora = 0;
    float s = 1.0f;
    int64_t max_tokens = 0;
    size_t ct = 2;                      // bytes of the compute type
    // adapter-derived, refreshed by prepare
    void* Ac = nullptr;                 // [r][in]   compute type
    void* At = nullptr;                 // [in][r]
    void* Bc = nullptr;                 // [out][r]
    void* Bt = nullptr;                 // [r][out]
    float* Pt = nullptr;                // [r][out]  (A W^T)
    float* G = nullptr;                 // [r][r]
    float* BG = nullptr;                // [out][r]  B G
    float* nsq = nullptr;               // [out]
    float* d = nullptr;                 // [out]
    const float* B = nullptr;           // adapter pointers of the last prepare (device)
    const float* mag = nullptr;
    // saved by forward for backward
    void* Hc = nullptr;                 // [max_tokens][r] compute type: s X A^T
    void* U = nullptr;                  // [max_tokens][out] compute type: pre-scale output
    int64_t saved_tokens = -1;
    // backward scratch
    void* dU = nullptr;                 // [max_tokens][out] compute type
    void* sdUB = nullptr;               // [max_tokens][r] compute type
    void* Xb = nullptr;                 // [max_tokens][in] bf16 copy of an f32 input (bf16 precision)
    float* gd = nullptr;                // [out]
    float* gn = nullptr;                // [out]
    void* Ax = nullptr;                 // [r][out] compute type: 2s (B*gn)^T
    void* A2x = nullptr;                // [r][r]   compute type: 2s^2 B^T diag(gn) B
    float* red = nullptr;               // [out][r] reduced dU^T Hc
    const char* tag = nullptr;          // role name for profiler scopes (lin_set_tag)
    // a member of a stacked product (lin_stack_*): U and Hc are column slices of the stack's outputs
    // with these row strides; the buffers named in `ext` belong to the stack
    int64_t ldu = 0, ldh = 0;
    unsigned ext = 0;
    // merged mode (bf16 precision): the products contract W_eff = W + s B A, refreshed by prepare
    int merged = 0;
    void* Wm = nullptr;                 // [out][in] bf16 W_eff
    void* Wmt = nullptr;                // [in][out] bf16 W_eff^T
    sa3k::LinGroup* solo = nullptr;     // one-member group refreshing a separately prepared linear
    const float* solo_key[4] = {};      // its A, B, magnitude, base_norm_sq pointers
    float solo_s = 0.0f;
    int solo_dora = -1;
};

namespace {

constexpr int kThreads = 256;

// "<base>.<tag>" while profiling a tagged linear, else base; names are interned (scopes keep the pointer)
const char* scope(const sa3k_ctx* ctx, const sa3k_lin* L, const char* base) {
    if (!ctx->prof_on || !L->tag) return base;
    static std::set<std::string> names;
    return names.insert(std::string(base) + "." + L->tag).first->c_str();
}

template <class T>
T* dev_alloc(size_t n) {
    void* p = nullptr;
    if (n == 0) n = 1;
    SA3K_HIP(hipMalloc(&p, n * sizeof(T)));
    return static_cast<T*>(p);
}

// ---------------------------------------------------------------- weight layout
// transpose a [rows][cols] matrix of T into [cols][rows] through a 32x32 LDS tile
template <class T>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                              int64_t rows, int64_t cols) {
    __shared__ T tile[32][33];
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
    for (int k = ty; k < 32; k += 8) {
        const int64_t r = r0 + k, c = c0 + tx;
        if (r < rows && c < cols) tile[k][tx] = src[r * cols + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (r < rows && c < cols) dst[c * rows + r] = tile[tx][k];
    }
}

template <class T>
void transpose(sa3k_ctx* ctx, const T* src, T* dst, int64_t rows, int64_t cols) {
    dim3 grid((unsigned)ceil_div(cols, 32), (unsigned)ceil_div(rows, 32));
    transpose_kernel<T><<<grid, kThreads, 0, ctx->stream>>>(src, dst, rows, cols);
    SA3K_LAUNCHED();
}

// Q8_0 blocks -> int8 quants [out][in] + f16 scales [out][in/32] (bytes copied, not re-encoded)
__global__ __launch_bounds__(kThreads) void q8_split_kernel(const uint16_t* __restrict__ blocks,
                                                            int8_t* __restrict__ qs, uint16_t* __restrict__ sc,
                                                            int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nb) return;
    const uint16_t* src = blocks + b * 17;
    sc[b] = src[0];
    uint16_t* dq = reinterpret_cast<uint16_t*>(qs + b * 32);
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[j] = src[1 + j];
}

__device__ inline float load_w(const sa3k_weight& w, const void* p, const void* ps, int64_t idx, int64_t in) {
    switch (w.type) {
        case SA3K_TYPE_F32: return static_cast<const float*>(p)[idx];
        case SA3K_TYPE_F16: return (float)static_cast<const _Float16*>(p)[idx];
        case SA3K_TYPE_BF16: return (float)static_cast<const bf16*>(p)[idx];
        default: {  // Q8_0 split: value = scale[row][col/32] * q
            const int64_t row = idx / in, col = idx - row * in;
            return (float)static_cast<const _Float16*>(ps)[row * (in / 32) + (col >> 5)] *
                   (float)static_cast<const int8_t*>(p)[idx];
        }
    }
}

// decoded bf16 copy of the forward layout (RNE of the exact decoded value)
__global__ __launch_bounds__(kThreads) void decode_bf16_kernel(sa3k_weight w, bf16* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= w.in * w.out) return;
    dst[i] = (bf16)load_w(w, w.w, w.ws, i, w.in);
}

// sum_i W[o][i]^2 in double per row; mode 0: + in*eps (nsq), mode 1: sqrt (norms)
__global__ __launch_bounds__(kThreads) void row_norm_kernel(sa3k_weight w, float eps, int mode,
                                                            float* __restrict__ out) {
    __shared__ double sh[kThreads / 64];
    const int64_t o = blockIdx.x;
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < w.in; i += kThreads) {
        const float v = load_w(w, w.w, w.ws, o * w.in + i, w.in);
        acc += (double)v * v;
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int k = 0; k < kThreads / 64; ++k) s += sh[k];
        out[o] = mode == 0 ? (float)(s + (double)w.in * eps) : (float)sqrt(s);
    }
}

// ---------------------------------------------------------------- adapter prepare
template <class CT>
__global__ __launch_bounds__(kThreads) void cvt_kernel(const float* __restrict__ src, CT* __restrict__ dst,
                                                       int64_t n, float scale) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) dst[i] = (CT)(src[i] * scale);
}

template <class CT>
__global__ __launch_bounds__(kThreads) void cvt_t_kernel(const float* __restrict__ src, CT* __restrict__ dst,
                                                         int64_t rows, int64_t cols) {
    // dst[c][r] = src[r][c] (small adapter matrices)
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i - r * cols;
    dst[c * rows + r] = (CT)src[i];
}

// G[a][b] = sum_i A[a][i] A[b][i] (one block per (a,b), double accumulation)
__global__ __launch_bounds__(kThreads) void gram_kernel(const float* __restrict__ A, int64_t in, int r,
                                                        float* __restrict__ G) {
    __shared__ double sh[kThreads / 64];
    const int a = blockIdx.x / r, b = blockIdx.x % r;
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < in; i += kThreads) acc += (double)A[a * in + i] * A[b * in + i];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) G[a * r + b] = (float)(sh[0] + sh[1] + sh[2] + sh[3]);
}

// per output row o: t2 = sum_a P[o][a] B[o][a]; BG[o] = B[o] G; t3 = B[o] . BG[o];
// nsq = bnsq + 2s t2 + s^2 t3; d = m / sqrt(nsq)
// One block = 8 output rows; thread (row, a) with a < 32 the rank index; the rank sums are
// 32-lane shuffles. G and the block's B rows are staged in LDS.
__global__ __launch_bounds__(kThreads) void dora_terms_kernel(const float* __restrict__ Pt, const float* __restrict__ B,
                                                              const float* __restrict__ G, const float* __restrict__ bnsq,
                                                              const float* __restrict__ mag, int64_t out, int r, float s,
                                                              float* __restrict__ BG, float* __restrict__ nsq,
                                                              float* __restrict__ d) {
    __shared__ float gs[32][33];
    __shared__ float bs[8][32];
    const int ol = threadIdx.x >> 5, a = threadIdx.x & 31;
    const int64_t o = (int64_t)blockIdx.x * 8 + ol;
    for (int k = threadIdx.x; k < 32 * 32; k += kThreads) {
        const int i = k >> 5, j = k & 31;
        gs[i][j] = (i < r && j < r) ? G[i * r + j] : 0.f;
    }
    bs[ol][a] = (o < out && a < r) ? B[o * r + a] : 0.f;
    __syncthreads();
    float g = 0.f;
#pragma unroll 8
    for (int c = 0; c < 32; ++c) g += bs[ol][c] * gs[c][a];
    float t2 = 0.f, t3 = 0.f;
    if (o < out && a < r) {
        BG[o * r + a] = g;
        t2 = Pt[(int64_t)a * out + o] * bs[ol][a];
        t3 = bs[ol][a] * g;
    }
    for (int off = 16; off > 0; off >>= 1) {
        t2 += __shfl_xor(t2, off, 32);
        t3 += __shfl_xor(t3, off, 32);
    }
    if (a == 0 && o < out) {
        const float n2 = bnsq[o] + 2.0f * s * t2 + s * s * t3;
        nsq[o] = n2;
        d[o] = mag[o] / sqrtf(n2);
    }
}

// ---------------------------------------------------------------- K3 column reductions
template <class CT>
__device__ inline float ld_ct(const CT* p, int64_t i) { return (float)p[i]; }

// Stage rows [nb, nb + cnt) of a [tokens][r] rank matrix into sh[64][R] (rows past cnt and ranks
// past r read as 0). Every thread's loads are issued before the first LDS write: one memory round
// trip per 64-row chunk.
template <class CT, int R>
__device__ inline void stage_rank_rows(float (*sh)[R], const CT* __restrict__ P, int64_t nb, int cnt, int r) {
    constexpr int kPer = 64 * R / kThreads;
    static_assert(64 * R % kThreads == 0, "whole staging rounds");
    float v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int k = threadIdx.x + j * kThreads, row = k / R, a = k % R;
        v[j] = (row < cnt && a < r) ? ld_ct(P, (nb + row) * r + a) : 0.f;
    }
    __syncthreads();   // the previous chunk's readers are done
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int k = threadIdx.x + j * kThreads;
        sh[k / R][k % R] = v[j];
    }
    __syncthreads();
}

// token rows whose loads one thread issues before their sums (one memory round trip per batch)
constexpr int kColBatch = 32;

// Rows [r0, r1) of dY: dU = dY*d (stored, compute type), partial gd = sum dY*U and
// partial (dU^T Hc)[o][a] = sum_n dU[n][o] Hc[n][a]. One thread per column o.
template <class CT, int R>
__global__ __launch_bounds__(kThreads) void colred_dy_kernel(const float* __restrict__ dY, const CT* __restrict__ U,
                                                             const float* __restrict__ d, const CT* __restrict__ Hc,
                                                             CT* __restrict__ dU, float* __restrict__ part,
                                                             int64_t N, int64_t out, int r, int64_t rows_per) {
    __shared__ float hs[64][R];
    const int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per, r1 = min(N, r0 + rows_per);
    const float dd = (d && o < out) ? d[o] : 1.0f;
    float gd = 0.f, acc[R];
#pragma unroll
    for (int a = 0; a < R; ++a) acc[a] = 0.f;
    for (int64_t nb = r0; nb < r1; nb += 64) {
        const int cnt = (int)min((int64_t)64, r1 - nb);
        stage_rank_rows<CT, R>(hs, Hc, nb, cnt, r);
        if (o < out) {
            // the sums keep the row order
            for (int row0 = 0; row0 < cnt; row0 += kColBatch) {
                float y[kColBatch], u[kColBatch];
#pragma unroll
                for (int k = 0; k < kColBatch; ++k) {
                    const int64_t n = nb + min(row0 + k, cnt - 1);
                    y[k] = dY[n * out + o];
                    u[k] = U ? ld_ct(U, n * out + o) : 0.f;
                }
#pragma unroll
                for (int k = 0; k < kColBatch; ++k) {
                    const int row = row0 + k;
                    if (row < cnt) {
                        const float du = y[k] * dd;
                        if (U) gd += y[k] * u[k];
                        dU[(nb + row) * out + o] = (CT)du;
#pragma unroll
                        for (int a = 0; a < R; ++a) acc[a] += du * hs[row][a];
                    }
                }
            }
        }
    }
    if (o >= out) return;
    // partial layout: [split][R+1][out] (coalesced over o)
    float* p = part + (int64_t)blockIdx.y * (R + 1) * out;
    p[o] = gd;
#pragma unroll
    for (int a = 0; a < R; ++a) p[(int64_t)(a + 1) * out + o] = acc[a];
}

// partial (G^T X)[a][i] = sum_n G[n][a] X[n][i] over rows [r0, r1). One thread per column i.
template <class XT, class CT, int R>
__global__ __launch_bounds__(kThreads) void colred_x_kernel(const XT* __restrict__ X, const CT* __restrict__ Gm,
                                                            float* __restrict__ part, int64_t N, int64_t in, int r,
                                                            int64_t rows_per) {
    __shared__ float gs[64][R];
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per, r1 = min(N, r0 + rows_per);
    float acc[R];
#pragma unroll
    for (int a = 0; a < R; ++a) acc[a] = 0.f;
    for (int64_t nb = r0; nb < r1; nb += 64) {
        const int cnt = (int)min((int64_t)64, r1 - nb);
        stage_rank_rows<CT, R>(gs, Gm, nb, cnt, r);
        if (i < in) {
            for (int row0 = 0; row0 < cnt; row0 += kColBatch) {
                float x[kColBatch];
#pragma unroll
                for (int k = 0; k < kColBatch; ++k) x[k] = (float)X[(nb + min(row0 + k, cnt - 1)) * in + i];
#pragma unroll
                for (int k = 0; k < kColBatch; ++k) {
                    const int row = row0 + k;
                    if (row < cnt) {
#pragma unroll
                        for (int a = 0; a < R; ++a) acc[a] += x[k] * gs[row][a];
                    }
                }
            }
        }
    }
    if (i >= in) return;
    float* p = part + (int64_t)blockIdx.y * R * in;
#pragma unroll
    for (int a = 0; a < R; ++a) p[(int64_t)a * in + i] = acc[a];
}

// ---- the same column reductions on bf16 MFMA (bf16 precision): skinny "TN" products over tokens
//   TN_DY: Q = dU = dY * d (written out as bf16), part[z][0][c] = sum_n dY*U, part[z][1+a][c] =
//          sum_n Hc[n][a] dU[n][c]                                   (dU^T Hc, stride 33 rows)
//   TN_X:  part[z][a][c] = sum_n G[n][a] X[n][c]                      ((s dU B)^T X, stride 32 rows)
//   TN_DU: as TN_DY with Q = dU already written by the producer of dY: part[z][0][c] =
//          (sum_n dU*U) / d[c], part[z][1+a][c] = sum_n Hc[n][a] dU[n][c]
// over the token rows of split z. A workgroup owns 64 columns; per 32-token step the Q tile (dU or
// X, 32 tokens x 64 columns) and the P tile (Hc or G, 32 tokens x rank padded to 32) are stored
// row-major in LDS with 16- / 8-byte writes and read back with ds_read_b64_tr_b16, which hands
// each lane 4 consecutive tokens of one column: two of them make the 8-token MFMA operand. Each
// wave owns 16 columns x 32 ranks (two v_mfma_f32_16x16x32_bf16 per step). Two LDS buffers and
// the next step's global loads issued before the current step's LDS traffic keep the stream of
// Q in flight; the kernel is bound by streaming Q once.
constexpr int TN_DY = 0, TN_X = 1, TN_DU = 2;
constexpr int TN_COLS = 64, TN_ROWS = 32;
constexpr int TN_H = 2;                    // 32-token halves per step (each thread loads TN_H token rows)
constexpr int TN_STEP = TN_ROWS * TN_H;    // tokens per step (one barrier per step)
constexpr int TN_QLD = 144;   // bytes per token row of the Q tile (128 + 16: the four rows a transposed read touches sit in distinct banks)
constexpr int TN_PLD = 80;    // bytes per token row of the P tile (64 + 16)

typedef short tn_v4s __attribute__((ext_vector_type(4)));
typedef __bf16 tn_bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
// T[k0 .. k0+3][n0 + (lane%16)] of a row-major bf16 LDS tile with `ld` bytes per row (every 16-lane
// group of the wave may use its own k0, n0)
__device__ __forceinline__ tn_bf16x4 tn_ld_tr(const char* t, int ld, int k0, int n0, int lane) {
    const int j = lane & 15;
    const char* a = t + (k0 + (j >> 2)) * ld + (n0 + 4 * (j & 3)) * 2;
    return __builtin_bit_cast(tn_bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                               (__attribute__((address_space(3))) tn_v4s*)(
                                                   (__attribute__((address_space(3))) void*)a)));
}

__device__ __forceinline__ bf16x8 cat44(tn_bf16x4 a, tn_bf16x4 b) {
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// The per-output-row step that follows the dY column reduction of an adapted linear (the rows
// kernel's formulas, dora_bwd_rows_kernel below), run by the reduction's last split to arrive when
// dB is set.
struct RowsArgs {
    const float *nsq, *mag, *Pt, *BG, *B;
    float s;
    int dora;
    float *dB, *dm, *gn;
    bf16* Ax;
};

template <int MODE, class QT>
__global__ __launch_bounds__(kThreads) void skinny_tn_kernel(const QT* __restrict__ Q, const bf16* __restrict__ P, int r,
                                                             const bf16* __restrict__ U, const float* __restrict__ d,
                                                             bf16* __restrict__ dU, float* __restrict__ part, int64_t N,
                                                             int64_t cols, int64_t rows_per, float* __restrict__ out,
                                                             int accumulate, int* __restrict__ counters, RowsArgs rows,
                                                             int64_t ldu, int64_t ldp) {
    // ldu / ldp: row strides of U and P in elements (the rows of a wider matrix); Q has `cols`
    __shared__ __attribute__((aligned(16))) char qt[2][TN_STEP * TN_QLD];
    __shared__ __attribute__((aligned(16))) char pt[2][TN_STEP * TN_PLD];
    __shared__ float red[TN_ROWS][TN_COLS + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t c0 = (int64_t)blockIdx.x * TN_COLS;
    const int z = blockIdx.y;
    const int64_t r0 = (int64_t)z * rows_per, r1 = min(N, r0 + rows_per);
    const int lrow = tid >> 3;            // token row of this thread's loads within a step half
    const int c8 = (tid & 7) * 8;         // its 8 columns
    const int a4 = (tid & 7) * 4;         // its 4 ranks of the P tile
    const int64_t col = c0 + c8;
    const bool col_ok = col < cols;       // cols is a multiple of 8
    float dd[8], gd[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        gd[j] = 0.f;
        dd[j] = (MODE == TN_DY && d && col_ok) ? d[col + j] : 1.0f;
    }
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const int g = lane >> 4;

    // one step's global operands of this thread, loaded ahead of use
    struct Regs {
        float4 ya[TN_H], yb[TN_H];   // dY (DY) or f32 X
        bf16x8 u[TN_H];              // U (DY, DU) or bf16 X
        bf16x8 q[TN_H];              // dU (DU)
        uint2 pv[TN_H];              // 4 bf16 of P
    };
    // Loads through buffer descriptors whose extents end at this split's last token row: rows past
    // it, absent U (extent 0) and columns past the end (offset beyond every extent) read as zeros
    // with no branch, so the loads of a step are one straight run the wait counter can track.
    typedef unsigned tn_v4u __attribute__((ext_vector_type(4)));
    typedef unsigned tn_v2u __attribute__((ext_vector_type(2)));
    constexpr uint32_t kOut = 0xFFFFFFF0u;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<QT*>(Q), (short)0, (int)(r1 * cols * (int64_t)sizeof(QT)), 0x00020000);
    constexpr bool kGd = MODE == TN_DY || MODE == TN_DU;   // the magnitude column sums gd
    const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(kGd && U ? U : static_cast<const bf16*>(nullptr)), (short)0,
        (kGd && U) ? (int)(r1 * ldu * 2) : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(P), (short)0,
                                                                        (int)(r1 * ldp * 2), 0x00020000);
    auto load = [&](int64_t n0, Regs& R) {
#pragma unroll
        for (int h = 0; h < TN_H; ++h) {
            const int64_t n = n0 + lrow + TN_ROWS * h;
            const uint32_t e = col_ok ? (uint32_t)(n * cols + col) : 0u;   // element offset of the 8 columns
            const uint32_t eu = col_ok ? (uint32_t)(n * ldu + col) : 0u;   // the same in U
            const uint32_t pe = a4 < r ? (uint32_t)(n * ldp + a4) : 0u;
            if constexpr (MODE == TN_DY || sizeof(QT) == 4) {
                const uint32_t off = col_ok ? e * 4u : kOut;
                R.ya[h] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
                R.yb[h] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, off + 16u, 0, 0));
            }
            if constexpr (MODE == TN_DY) {
                R.u[h] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ru, col_ok ? eu * 2u : kOut, 0, 0));
            } else if constexpr (MODE == TN_DU) {
                R.q[h] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, col_ok ? e * 2u : kOut, 0, 0));
                R.u[h] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(ru, col_ok ? eu * 2u : kOut, 0, 0));
            } else if constexpr (sizeof(QT) == 2) {
                R.u[h] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, col_ok ? e * 2u : kOut, 0, 0));
            }
            R.pv[h] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rp, a4 < r ? pe * 2u : kOut, 0, 0));
        }
    };
    // LDS tiles of one step (and, DY, dU out + the gd partials)
    auto stage = [&](int64_t n0, const Regs& R, int b) {
#pragma unroll
        for (int h = 0; h < TN_H; ++h) {
            const int64_t n = n0 + lrow + TN_ROWS * h;
            bf16x8 qv;
            if constexpr (MODE == TN_DY) {
                const float y[8] = {R.ya[h].x, R.ya[h].y, R.ya[h].z, R.ya[h].w,
                                    R.yb[h].x, R.yb[h].y, R.yb[h].z, R.yb[h].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float q = y[j] * dd[j];
                    qv[j] = (bf16)q;
                    if (U) gd[j] += y[j] * (float)R.u[h][j];
                }
                if (n < r1 && col_ok) *reinterpret_cast<bf16x8*>(dU + n * cols + col) = qv;
            } else if constexpr (MODE == TN_DU) {
                qv = R.q[h];
                if (U) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) gd[j] += (float)qv[j] * (float)R.u[h][j];
                }
            } else if constexpr (sizeof(QT) == 4) {
                const float y[8] = {R.ya[h].x, R.ya[h].y, R.ya[h].z, R.ya[h].w,
                                    R.yb[h].x, R.yb[h].y, R.yb[h].z, R.yb[h].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) qv[j] = (bf16)y[j];
            } else {
                qv = R.u[h];
            }
            const int lr = lrow + TN_ROWS * h;
            *reinterpret_cast<bf16x8*>(qt[b] + lr * TN_QLD + c8 * 2) = qv;
            *reinterpret_cast<uint2*>(pt[b] + lr * TN_PLD + a4 * 2) = R.pv[h];
        }
    };
    // D[i][j] += sum over the step's tokens: i = column wave*16 + 4g+v, j = rank t*16 + lane%16
    auto mma = [&](int b) {
#pragma unroll
        for (int h = 0; h < TN_H; ++h) {
            const int k0 = TN_ROWS * h + 8 * g;
            const bf16x8 af = cat44(tn_ld_tr(qt[b], TN_QLD, k0, wave * 16, lane),
                                    tn_ld_tr(qt[b], TN_QLD, k0 + 4, wave * 16, lane));
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf16x8 bfr = cat44(tn_ld_tr(pt[b], TN_PLD, k0, t * 16, lane),
                                         tn_ld_tr(pt[b], TN_PLD, k0 + 4, t * 16, lane));
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr, acc[t], 0, 0, 0);
            }
        }
    };

    // Two register sets, the loop unrolled by two steps: while step n0 is staged from set A, set B
    // holds step n0 + TN_STEP in flight, and A is refilled with step n0 + 2 TN_STEP right after its
    // stage. The loads are issued unconditionally (rows past the split read zeros), so the
    // compiler's wait before each stage counts only the other set's loads.
    Regs ra, rb;
    load(r0, ra);
    load(r0 + TN_STEP, rb);
    for (int64_t n0 = r0; n0 < r1; n0 += 2 * TN_STEP) {
        stage(n0, ra, 0);
        __syncthreads();   // step n0 in buffer 0; every wave is done with buffer 0's previous use
        mma(0);
        load(n0 + 2 * TN_STEP, ra);
        if (n0 + TN_STEP >= r1) break;
        stage(n0 + TN_STEP, rb, 1);
        __syncthreads();
        mma(1);
        load(n0 + 3 * TN_STEP, rb);
    }
    // D[i][j]: i = column 4g + v of this wave's 16, j = rank t*16 + lane%16. The tile goes through
    // LDS (the Q staging buffer, free after the loop) so that every thread stores a whole 16-byte run
    // of a partial row: each 64-byte segment is written once and whole, which the device-coherent
    // (write-through) stores of the in-kernel reduction need to stay cheap.
    constexpr int RS = kGd ? 33 : 32;
    const int row0 = kGd ? 1 : 0;
    const int r16 = lane & 15;
    constexpr int TP = TN_COLS + 4;   // LDS tile pitch in floats (16-byte aligned rows)
    static_assert(32 * TP * 4 <= TN_STEP * TN_QLD, "partial tile does not fit the Q staging buffer");
    float* tile = reinterpret_cast<float*>(qt[0]);
    const __amdgpu_buffer_rsrc_t rpart = __builtin_amdgcn_make_buffer_rsrc(
        part, (short)0, (int)((int64_t)gridDim.y * RS * cols * 4), 0x00020000);
    __syncthreads();   // every wave is done with the Q tiles
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) tile[(t * 16 + r16) * TP + wave * 16 + 4 * g + v] = acc[t][v];
    if constexpr (kGd) {   // gd: the 32 token-row slots of each column
#pragma unroll
        for (int j = 0; j < 8; ++j) red[lrow][c8 + j] = gd[j];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {   // 16 threads per rank row, 4 columns each
        const int a = h * 16 + tid / 16, cc = (tid % 16) * 4;
        const int64_t c = c0 + cc;
        if (a < r && c < cols) {
            const float4 v = *reinterpret_cast<const float4*>(tile + a * TP + cc);
            const int64_t e = ((int64_t)z * RS + row0 + a) * cols + c;
            if (counters)   // read by the last split in this launch
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(tn_v4u, v), rpart, (uint32_t)(e * 4), 0, kSc1);
            else
                *reinterpret_cast<float4*>(part + e) = v;
        }
    }
    if constexpr (kGd) {
        if (tid < TN_COLS) {
            float s = 0.f;
            for (int k = 0; k < TN_ROWS; ++k) s += red[k][tid];
            if (c0 + tid < cols) {
                if (MODE == TN_DU && d) s = s / d[c0 + tid];   // sum dU U = d sum dY U
                float* dst = part + ((int64_t)z * RS) * cols + c0 + tid;
                if (counters) st_coherent(dst, s);
                else *dst = s;
            }
        }
    }
    if (!counters) return;   // reduced by the consumer (rows kernel) or sum_splits_kernel
    // The last split of this column tile to arrive sums the partials in split order
    // (deterministic) into out[row][c] (= or +=), or runs the rows step on them; nobody waits for
    // anybody.
    __shared__ int s_last;
    const uint32_t zstride = (uint32_t)(RS * cols * 4);
    if constexpr (kGd) {
        if (rows.dB) {
            // thread (column c0 + tid % 64, ranks tid / 64 + 4 i): the rows kernel's sums (split
            // order, from zero) and formulas, so the results are the same bit for bit. Its inputs
            // are loaded before the arrival (every split), so the last one's tail waits only for
            // the partial sums; every thread sums its column's gd itself (no barrier).
            constexpr int NG = kThreads / TN_COLS, NR = 32 / NG;
            const int cl = tid & (TN_COLS - 1), ag = tid / TN_COLS;
            const int64_t o = c0 + cl;
            const bool ok = o < cols;
            const int64_t oc = ok ? o : 0;
            const float n2 = rows.dora ? rows.nsq[oc] : 1.f, mg = rows.dora ? rows.mag[oc] : 0.f;
            float pt[NR], bb[NR], bg[NR], db[NR];
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const int a = min(ag + NG * i, r - 1);
                pt[i] = rows.dora ? rows.Pt[(int64_t)a * cols + oc] : 0.f;
                bb[i] = rows.dora ? rows.B[oc * r + a] : 0.f;
                bg[i] = rows.dora && rows.BG ? rows.BG[oc * r + a] : 0.f;
                db[i] = rows.dB[oc * r + a];
            }
            if (!arrive_last(&counters[blockIdx.x], (int)gridDim.y, &s_last)) return;
            const int splits = (int)gridDim.y;
            uint32_t off[NR + 1];
            float sum[NR + 1];
            off[0] = ok ? (uint32_t)(o * 4) : kOut;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const int a = ag + NG * i;
                off[1 + i] = ok && a < r ? (uint32_t)(((int64_t)(a + 1) * cols + o) * 4) : kOut;
            }
            coherent_split_sums(rpart, off, zstride, splits, sum);
            if (!ok) return;
            float gn = 0.f;
            if (rows.dora) {
                const float gs = sum[0];
                const float sq = sqrtf(n2);
                gn = -0.5f * gs * mg / (n2 * sq);
                if (ag == 0) {
                    if (rows.dm) rows.dm[o] += gs / sq;
                    rows.gn[o] = gn;
                }
            }
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const int a = ag + NG * i;
                if (a >= r) break;
                float v = sum[1 + i];
                if (rows.dora) {
                    v += 2.0f * rows.s * gn * pt[i];
                    if (rows.BG) v += 2.0f * rows.s * rows.s * gn * bg[i];
                    rows.Ax[(int64_t)a * cols + o] = (bf16)(2.0f * rows.s * bb[i] * gn);
                }
                rows.dB[o * r + a] = db[i] + v;
            }
            return;
        }
    }
    if (!arrive_last(&counters[blockIdx.x], (int)gridDim.y, &s_last)) return;
    const int splits = (int)gridDim.y;
    // element e = tid + kThreads k of the (rows x 64) tile: row e / 64, column c0 + e % 64
    constexpr int NE = (RS * TN_COLS + kThreads - 1) / kThreads;
    const int nrows = kGd ? r + 1 : r;
    uint32_t off[NE];
    float sum[NE];
#pragma unroll
    for (int k = 0; k < NE; ++k) {
        const int e = tid + kThreads * k, row = e / TN_COLS;
        const int64_t c = c0 + (e % TN_COLS);
        off[k] = row < nrows && c < cols ? (uint32_t)(((int64_t)row * cols + c) * 4) : kOut;
    }
    coherent_split_sums(rpart, off, zstride, splits, sum);
#pragma unroll
    for (int k = 0; k < NE; ++k) {
        const int e = tid + kThreads * k, row = e / TN_COLS;
        const int64_t c = c0 + (e % TN_COLS);
        if (row >= nrows || c >= cols) continue;
        float* o = out + (int64_t)row * cols + c;
        *o = accumulate ? *o + sum[k] : sum[k];
    }
}

// target workgroup count of a skinny TN reduction (environment SA3K_TN_WGS, for measurement)
int64_t ctx_tn_wgs() {
    static const int64_t v = [] {
        const char* e = std::getenv("SA3K_TN_WGS");
        return e ? std::max<int64_t>(64, std::atoll(e)) : (int64_t)0;
    }();
    return v;
}

// Token rows per split of a skinny TN reduction over `cols` columns. The launch has tiles x splits
// workgroups of 64 columns, up to 3 resident per CU (160 VGPRs, 37 KiB of LDS). Two of them on one
// CU overlap each other's memory latency; more share the CU's throughput. So a CU holding w of
// them takes about rows x max(1, w / 2) token rows of streaming time (8 bytes per element: dY or X,
// U, the dU store), and then each column tile's last split to arrive reads splits x rs x 64 partial
// sums (rs rows of partials), weighted 4: the partials' round trip through memory and the last
// split's wait cost more than their bytes at a CU's streaming rate (weights 2-6 measured equal on
// the DiT update, 0.2 ms under weight 1; 10 and more slower; environment SA3K_TN_RED overrides it,
// for measurement). The split count minimising the sum is taken; it keeps the busiest CU's load
// close to the average (576 workgroups over 256 CUs put 3 on some CUs and 2 on the rest). The same
// count serves the separate reduce launches (option tn_fuse 0), so both give the same sums.
int64_t tn_rows_per(int64_t cols, int64_t N, int rs) {
    const int64_t tiles = ceil_div(cols, TN_COLS);
    if (const int64_t w = ctx_tn_wgs())
        return std::max<int64_t>(TN_STEP, ceil_div(ceil_div(N * tiles, w), TN_STEP) * TN_STEP);
    constexpr int64_t kCUs = 256;
    int64_t best_rows = ceil_div(N, TN_STEP) * TN_STEP;
    double best = 1e300;
    for (int64_t S = 1; S <= 64; ++S) {
        const int64_t rows = std::max<int64_t>(2 * TN_STEP, ceil_div(ceil_div(N, S), TN_STEP) * TN_STEP);
        const int64_t splits = ceil_div(N, rows);
        const int64_t wgs = tiles * splits;
        if (ceil_div(wgs, kCUs) > 3 && S > 1) break;   // more than 3 resident per CU: no gain
        const double w = (double)ceil_div(wgs, kCUs);
        static const double red_scale = [] {
            const char* e = std::getenv("SA3K_TN_RED");
            return e ? std::atof(e) : 4.0;
        }();
        const double red = red_scale * (double)splits * rs * TN_COLS * 4.0;
        const double cost = std::max(1.0, w / 2.0) * (double)rows * TN_COLS * 8.0 + red;
        if (cost < best - 1e-9) {
            best = cost;
            best_rows = rows;
        }
    }
    return best_rows;
}

// partial sums of the column reductions: one buffer per context, shared by every linear (used
// in turn on the context stream); it grows outside graph capture only
float* reduce_workspace(sa3k_ctx* ctx, size_t bytes) {
    // one workspace per stream
    const bool side = ctx->stream == ctx->side_stream, quick = ctx->stream == ctx->quick_stream;
    void*& ws = side ? ctx->red_ws_side : quick ? ctx->red_ws_quick : ctx->red_ws;
    size_t& have = side ? ctx->red_ws_side_bytes : quick ? ctx->red_ws_quick_bytes : ctx->red_ws_bytes;
    if (bytes > have) {
        SA3K_REQUIRE(!ctx->capturing, "the reduction workspace cannot grow while a graph is being captured");
        if (ws) {
            SA3K_HIP(hipStreamSynchronize(ctx->stream));
            SA3K_HIP(hipFree(ws));
            ws = nullptr;
            have = 0;
        }
        SA3K_HIP(hipMalloc(&ws, bytes));
        have = bytes;
    }
    return static_cast<float*>(ws);
}

// y[j] (+)= sum_s part[s][j], j < n (fixed summation order: deterministic)
__global__ __launch_bounds__(kThreads) void sum_splits_kernel(const float* __restrict__ part, int64_t stride, int S,
                                                              int64_t n, float* __restrict__ y, int accumulate) {
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (j >= n) return;
    // eight splits' loads in flight at a time (past the last split: re-read, not added); the sums
    // are added in split order from zero
    float s = 0.f;
    for (int k0 = 0; k0 < S; k0 += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = part[(int64_t)min(k0 + k, S - 1) * stride + j];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k0 + k < S) s += v[k];
    }
    y[j] = accumulate ? y[j] + s : s;
}

// gd[o] and dUtH[a][o] are the split sums (in split order) of the column-reduction partials
// part[sp][row][o], row 0 = gd, row 1 + a = dUtH[a]; then
// dm += gd/sqrt(nsq); gn = -gd m nsq^-3/2 / 2; dB[o][a] += dUtH[a][o] + 2s gn P[o][a] + 2s^2 gn BG[o][a];
// Ax[a][o] = 2s B[o][a] gn[o]  (lora: dB += dUtH only). With BG null, P is W_eff A^T = P + s B G and
// the last term is left out.
template <class CT>
__global__ __launch_bounds__(kThreads) void dora_bwd_rows_kernel(const float* __restrict__ part, int S, int64_t stride,
                                                                 const float* __restrict__ nsq, const float* __restrict__ mag,
                                                                 const float* __restrict__ Pt, const float* __restrict__ BG,
                                                                 const float* __restrict__ B, int64_t out, int r, float s,
                                                                 int dora, float* __restrict__ dB, float* __restrict__ dm,
                                                                 float* __restrict__ gn_out, CT* __restrict__ Ax) {
    // thread (o, a): 64 consecutive output rows x 4 rank indices per block (o fastest, so the
    // partial sums read whole lines)
    const int64_t o = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    const int a = (int)blockIdx.y * 4 + (threadIdx.x >> 6);
    if (o >= out) return;
    float gn = 0.f;
    // split sums in split order; loads issued 8 at a time
    auto split_sum = [&](const float* p0) {
        float acc = 0.f;
        int sp = 0;
        for (; sp + 8 <= S; sp += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = p0[(int64_t)(sp + k) * stride];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc += v[k];
        }
        for (; sp < S; ++sp) acc += p0[(int64_t)sp * stride];
        return acc;
    };
    if (dora) {
        const float g = split_sum(part + o);
        const float n2 = nsq[o], sq = sqrtf(n2);
        gn = -0.5f * g * mag[o] / (n2 * sq);
        if (a == 0) {
            if (dm) dm[o] += g / sq;
            gn_out[o] = gn;
        }
    }
    if (a >= r) return;
    float v = split_sum(part + (int64_t)(a + 1) * out + o);
    if (dora) {
        v += 2.0f * s * gn * Pt[(int64_t)a * out + o];
        if (BG) v += 2.0f * s * s * gn * BG[o * r + a];   // null: Pt already holds W_eff A^T
        Ax[(int64_t)a * out + o] = (CT)(2.0f * s * B[o * r + a] * gn);
    }
    dB[o * r + a] += v;
}

// A2x[a][b] = 2 s^2 sum_o B[o][a] gn[o] B[o][b]  (one block per (a,b))
template <class CT>
__global__ __launch_bounds__(kThreads) void btgb_kernel(const float* __restrict__ B, const float* __restrict__ gn,
                                                        int64_t out, int r, float s, CT* __restrict__ A2x) {
    __shared__ float sh[kThreads / 64];
    const int a = blockIdx.x / r, b = blockIdx.x % r;
    float acc = 0.f;
    for (int64_t o = threadIdx.x; o < out; o += kThreads) acc += B[o * r + a] * gn[o] * B[o * r + b];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) A2x[a * r + b] = (CT)(2.0f * s * s * (sh[0] + sh[1] + sh[2] + sh[3]));
}

int src_of_weight(int type, bool transposed) {
    switch (type) {
        case SA3K_TYPE_F32: return SRC_F32;
        case SA3K_TYPE_F16: return SRC_F16;
        case SA3K_TYPE_BF16: return SRC_BF16;
        case SA3K_TYPE_Q8_0: return transposed ? SRC_Q8T : SRC_Q8;
    }
    sa3k_throw(SA3K_ERR_UNSUPPORTED, "weight type");
    return 0;
}

size_t type_size(int type) {
    switch (type) {
        case SA3K_TYPE_F32: return 4;
        case SA3K_TYPE_F16: case SA3K_TYPE_BF16: return 2;
        case SA3K_TYPE_Q8_0: return 1;
    }
    sa3k_throw(SA3K_ERR_UNSUPPORTED, "weight type");
    return 0;
}

void free_weight(sa3k_weight* w) {
    if (!w) return;
    for (void* p : {w->w, w->ws, w->wt, w->wts, w->wb, w->wbt}) if (p) (void)hipFree(p);
    delete w;
}

// buffers of a linear that a stacked product owns instead (sa3k_lin::ext)
constexpr unsigned kExtAc = 1, kExtD = 2, kExtWm = 4, kExtU = 8, kExtHc = 16;

void free_lin(sa3k_lin* L) {
    if (!L) return;
    if (L->solo) lin_group_free(L->solo);
    for (void* p : {L->Xb, L->At, L->Bc, L->Bt, (void*)L->Pt, (void*)L->G, (void*)L->BG, (void*)L->nsq, L->dU,
                    L->sdUB, (void*)L->gd, (void*)L->gn, L->Ax, L->A2x, (void*)L->red, L->Wmt})
        if (p) (void)hipFree(p);
    const std::pair<void*, unsigned> own[] = {{L->Ac, kExtAc}, {(void*)L->d, kExtD}, {L->Wm, kExtWm},
                                              {L->U, kExtU}, {L->Hc, kExtHc}};
    for (const auto& [p, bit] : own)
        if (p && !(L->ext & bit)) (void)hipFree(p);
    delete L;
}

// row split count for the column reductions: enough blocks to cover the chip
int choose_splits(int64_t cols, int64_t N) {
    // about 512 blocks in total, at least 64 rows per split (fewer partial sums to reduce)
    const int64_t col_blocks = ceil_div(cols, kThreads);
    int64_t S = ceil_div(512, col_blocks);
    S = std::max<int64_t>(1, std::min<int64_t>(S, ceil_div(N, 64)));
    return (int)std::min<int64_t>(S, 64);
}

struct WOp {
    int src;
    const void* p;
    const void* s;
    int64_t ld, lds;
};

// B operand of X W^T (transposed = false) or of dU W (transposed = true)
WOp weight_operand(const sa3k_weight* W, bool bf, bool transposed) {
    if (bf && W->wb) return transposed ? WOp{SRC_BF16, W->wbt, nullptr, W->out, 0} : WOp{SRC_BF16, W->wb, nullptr, W->in, 0};
    if (transposed) return WOp{src_of_weight(W->type, true), W->wt, W->wts, W->out, W->out};
    return WOp{src_of_weight(W->type, false), W->w, W->ws, W->in, W->in / 32};
}

// Epilogue work of the main product beyond Y: sw_g, the FFN SwiGLU g = bf16(val * silu(glu)) of Y =
// [val | glu], or hp, the attention heads prepared from Y, where the chosen kernel allows it (*done
// set to 1 then); Yb, a bf16 copy of Y, with Y itself written only where that work is not done.
struct LinEpi {
    bf16* sw_g = nullptr;
    const HeadPrep* hp = nullptr;
    bf16* Yb = nullptr;
    int* done = nullptr;
};

template <class CT>
void lin_forward_t(sa3k_ctx* ctx, sa3k_lin* L, int x_src, const void* X, int64_t N, const float* bias, float* Y,
                   const LinEpi* epi = nullptr) {
    SA3K_REQUIRE(L->ext == 0, "a linear of a stacked product runs its forward through the stack");
    const sa3k_weight* W = L->W;
    const bool bf = L->prec == SA3K_PREC_BF16;
    // merged: Hc feeds only the backward's dB reduction, so it is computed beside the main product
    const bool merged = L->merged && L->rank > 0;
    const bool side = merged && side_usable(ctx);
    if (bf && x_src == SRC_F32) {   // one pass to bf16 so both GEMMs stream compute-type operands
        const int64_t n = N * W->in;
        if (side) fork_arm(ctx);   // the conversion records the fork of the rank product
        KernelScope ks(ctx, scope(ctx, L, "lin_fwd_cvt_x"));
        launch_k(ctx, true, cvt_kernel<bf16>, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                 static_cast<const float*>(X), static_cast<bf16*>(L->Xb), n, 1.0f);
        SA3K_LAUNCHED();
        X = L->Xb;
        x_src = SRC_BF16;
    }
    // merged: Hc = s X A^T as r extra output columns of the main product (B rows from A) when they
    // cost it no extra round of workgroups, else as its own product beside it
    const bool h_cols = merged && bf && (ctx->rank_cols & 1) && gemm_extra_cols_free(ctx, N, W->out, W->in, L->rank);
    // Hc = s X A^T
    if (L->rank > 0 && !h_cols) {
        GemmDesc h;
        h.prec = L->prec; h.a_src = x_src; h.b_src = bf ? SRC_BF16 : SRC_F32;
        h.A = X; h.lda = W->in; h.B = L->Ac; h.ldb = W->in;
        h.M = N; h.N = L->rank; h.K = W->in; h.alpha = L->s;
        if (bf) { h.Cb = static_cast<bf16*>(L->Hc); h.ldcb = L->rank; }
        else { h.C = static_cast<float*>(L->Hc); h.ldc = L->rank; }
        if (side) fork_fire(ctx);   // X is ready
        OnSide os(ctx, side);
        gemm_run(ctx, h, scope(ctx, L, "lin_fwd_h"));
    }
    GemmDesc g;
    g.prec = L->prec; g.a_src = x_src;
    g.A = X; g.lda = W->in;
    if (merged) {   // Y = d (.) (X W_eff^T) + bias
        g.b_src = SRC_BF16; g.B = L->Wm; g.ldb = W->in;
        if (h_cols) { g.Nx = L->rank; g.Bx = L->Ac; g.ldbx = W->in; g.alpha_x = L->s; g.Cbn = static_cast<bf16*>(L->Hc); g.ldcn = L->rank; }
    } else {        // Y = d (.) (X W^T + Hc B^T) + bias: the rank term as the second segment
        const WOp wo = weight_operand(W, bf, false);
        g.b_src = wo.src; g.B = wo.p; g.ldb = wo.ld; g.Bs = wo.s; g.ldbs = wo.lds;
        if (L->rank > 0) { g.A2 = L->Hc; g.lda2 = L->rank; g.B2 = L->Bc; g.ldb2 = L->rank; g.K2 = L->rank; }
    }
    g.M = N; g.N = W->out; g.K = W->in; g.alpha = 1.0f;
    g.colscale = L->dora ? L->d : nullptr;
    g.bias = bias;
    g.C = Y; g.ldc = W->out;
    g.ldu = W->out;
    if (L->dora) { if (bf) g.Ub = static_cast<bf16*>(L->U); else g.U = static_cast<float*>(L->U); }
    if (epi) {
        if (epi->sw_g && W->out % 2 == 0) {
            g.sw_half = W->out / 2; g.sw_g = epi->sw_g; g.sw_ldg = W->out / 2; g.sw_done = epi->done;
        }
        if (epi->hp) { g.hp = *epi->hp; g.hp_done = epi->done; }
        if (epi->Yb) { g.Cb = epi->Yb; g.ldcb = W->out; g.c_unfused_only = 1; }
    }
    gemm_run(ctx, g, scope(ctx, L, "lin_fwd_main"));
    if (side) side_join_unless_deferred(ctx);
    L->saved_tokens = N;
}

// dY null: the producer of the output gradient has written dU = bf16(d (.) dY) (d = 1 without
// DoRA) into L->dU itself (bf16 precision only)
template <class CT, int R>
void lin_backward_t(sa3k_ctx* ctx, sa3k_lin* L, int x_src, const void* X, int64_t N, const float* dY, float* dX,
                    int dx_acc, float* dA, float* dB, float* dm, const DxEpi* epi = nullptr) {
    const sa3k_weight* W = L->W;
    const bool bf = L->prec == SA3K_PREC_BF16;
    const int64_t in = W->in, out = W->out;
    const int r = L->rank;
    const bool du_ready = dY == nullptr;
    SA3K_REQUIRE(!du_ready || sizeof(CT) == 2, "a precomputed dU needs bf16 precision");
    if (r == 0) {   // plain mul_mat: dX = dY W only
        if (!dX) return;
        const void* dyc = du_ready ? L->dU : dY;
        if (bf && !du_ready) {
            const int64_t n = N * out;
            KernelScope ks(ctx, scope(ctx, L, "lin_bwd_cvt_dy"));
            cvt_kernel<bf16><<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(dY, static_cast<bf16*>(L->dU),
                                                                                        n, 1.0f);
            SA3K_LAUNCHED();
            dyc = L->dU;
        }
        const WOp wt = weight_operand(W, bf, true);
        GemmDesc g;
        g.prec = L->prec; g.a_src = bf ? SRC_BF16 : SRC_F32; g.b_src = wt.src;
        g.A = dyc; g.lda = out; g.B = wt.p; g.ldb = wt.ld; g.Bs = wt.s; g.ldbs = wt.lds;
        g.M = N; g.N = in; g.K = out; g.alpha = 1.0f;
        g.C = dX; g.ldc = in; g.accumulate = dx_acc;
        if (epi) { g.ad = epi->ad; g.sb = epi->sb; g.bwd_done = epi->done; }
        gemm_run(ctx, g, scope(ctx, L, "lin_bwd_dx"));
        return;
    }
    const bool merged = L->merged && sizeof(CT) == 2;
    const bool side = side_usable(ctx);
    // the dA column reduction X^T sdUB: its split partials summed by its own last split to arrive
    // (option tn_fuse, or gemm_fixup) or by a separate launch
    int64_t x_rows_per = 0;
    int x_S = 0;
    bool x_fused = false;
    if constexpr (sizeof(CT) == 2) {
        const int64_t x_tiles = ceil_div(in, TN_COLS);
        x_fused = tn_counters(ctx, x_tiles, kFuseXSum) != nullptr || use_fixup(ctx, (int64_t)32 * in, x_tiles);
        x_rows_per = tn_rows_per(in, N, 32);
        x_S = (int)ceil_div(N, x_rows_per);
    } else {
        x_S = choose_splits(in, N);
        x_rows_per = ceil_div(N, x_S);
    }
    bool rows_fused = false;   // the rows step runs in the column reduction's last split
    // row strides of the saved U and Hc (wider when a stacked product wrote them)
    const int64_t ldu = L->ldu ? L->ldu : out, ldh = L->ldh ? L->ldh : r;
    // 1. dU = dY*d, gd, dU^T Hc (column reduction over tokens); the split partials rp[rS][rows][out]
    const float* rp = nullptr;
    int rS = 1;
    int64_t rstride = 0;
    if constexpr (sizeof(CT) == 2) {
        // the skinny TN kernels address dY / X through 32-bit buffer offsets (with a few steps of
        // look-ahead past the last token row)
        SA3K_REQUIRE((N + 4 * TN_STEP) * std::max(std::max(in, out), ldu) * 4 < ((int64_t)1 << 32),
                     "tokens x features too large for one adapted-linear backward");
        // tn_fuse: the reduction's last split per column tile runs the rows step itself; else
        // (gemm_fixup) it sums the partials into L->red for the rows kernel, or that kernel sums them
        int* counters = tn_counters(ctx, ceil_div(out, TN_COLS), kFuseRows);
        rows_fused = counters != nullptr;
        if (!counters && use_fixup(ctx, (int64_t)33 * out, ceil_div(out, TN_COLS))) counters = stream_counters(ctx);
        const int64_t rows_per = tn_rows_per(out, N, 33);
        const int S = (int)ceil_div(N, rows_per);
        float* part = reduce_workspace(ctx, (size_t)S * 33 * out * sizeof(float));
        RowsArgs ra{};
        if (rows_fused)
            ra = RowsArgs{L->nsq, L->mag, L->Pt, L->merged ? nullptr : L->BG, L->B, L->s, L->dora, dB, dm, L->gn,
                          static_cast<bf16*>(L->Ax)};
        if (rows_fused && side && L->merged) fork_arm(ctx);   // recorded by this kernel: dU and Ax ready
        {
            KernelScope ks(ctx, scope(ctx, L, "lin_bwd_colred_dy"), 2.0 * N * out * r);
            const dim3 grid((unsigned)ceil_div(out, TN_COLS), (unsigned)S);
            if (du_ready)
                launch_k(ctx, true, skinny_tn_kernel<TN_DU, bf16>, grid, dim3(kThreads), 0,
                         static_cast<const bf16*>(L->dU), static_cast<const bf16*>(L->Hc), r,
                         static_cast<const bf16*>(L->dora ? L->U : nullptr), (const float*)(L->dora ? L->d : nullptr),
                         (bf16*)nullptr, part, N, out, rows_per, L->red, 0, counters, ra, ldu, ldh);
            else
                launch_k(ctx, true, skinny_tn_kernel<TN_DY, float>, grid, dim3(kThreads), 0, dY,
                         static_cast<const bf16*>(L->Hc), r, static_cast<const bf16*>(L->dora ? L->U : nullptr),
                         (const float*)(L->dora ? L->d : nullptr), static_cast<bf16*>(L->dU), part, N, out, rows_per,
                         L->red, 0, counters, ra, ldu, ldh);
            SA3K_LAUNCHED();
        }
        // the rows kernel below sums the S partials (or, after the in-kernel reduction, reads the
        // one sum in L->red)
        if (counters) { rp = L->red; rS = 1; }
        else { rp = part; rS = S; }
        rstride = (int64_t)33 * out;
    } else {
        const int S = choose_splits(out, N);
        const int64_t rows_per = ceil_div(N, S);
        float* part = reduce_workspace(ctx, (size_t)S * (R + 1) * out * sizeof(float));
        dim3 grid((unsigned)ceil_div(out, kThreads), (unsigned)S);
        {
            KernelScope ks(ctx, scope(ctx, L, "lin_bwd_colred_dy"));
            colred_dy_kernel<CT, R><<<grid, kThreads, 0, ctx->stream>>>(
                dY, static_cast<const CT*>(L->dora ? L->U : nullptr), L->dora ? L->d : nullptr,
                static_cast<const CT*>(L->Hc), static_cast<CT*>(L->dU), part, N, out, r, rows_per);
            SA3K_LAUNCHED();
        }
        rp = part; rS = S; rstride = (int64_t)(R + 1) * out;
    }
    // merged: the rows step's outputs (Ax) are the last inputs of the dX GEMM, and sdUB with its
    // column reduction only feeds dA: they go to the second stream as soon as dU and Ax are ready
    if (!rows_fused) {
        if (side && merged) fork_arm(ctx);   // recorded by the rows kernel
        KernelScope ks(ctx, scope(ctx, L, "lin_bwd_rows"));
        const dim3 grid((unsigned)ceil_div(out, 64), (unsigned)ceil_div(std::max(r, 1), 4));
        // merged: Pt holds W_eff A^T = P + s B G, so the B G term is already in it
        launch_k(ctx, true, dora_bwd_rows_kernel<CT>, grid, dim3(kThreads), 0, rp, rS, rstride,
                 (const float*)L->nsq, (const float*)L->mag, (const float*)L->Pt,
                 (const float*)(merged ? nullptr : L->BG), L->B, out, r, L->s, L->dora, dB, dm, L->gn,
                 static_cast<CT*>(L->Ax));
        SA3K_LAUNCHED();
    }
    // 2. sdUB = s dU B; dora: A2x = 2 s^2 B^T diag(gn) B = s * (Ax . Bt^T) contracts the same Bt
    //    over out, so it rides on the same GEMM as r extra rows (not needed when merged)
    const bool fold_btgb = L->dora && !merged && out % (bf ? 64 : 32) == 0;
    if (L->dora && !merged && !fold_btgb) {
        KernelScope ks(ctx, scope(ctx, L, "lin_bwd_btgb"));
        btgb_kernel<CT><<<(unsigned)(r * r), kThreads, 0, ctx->stream>>>(L->B, L->gn, out, r, L->s,
                                                                         static_cast<CT*>(L->A2x));
        SA3K_LAUNCHED();
    }
    float* x_part = nullptr;
    // the partials go to the second stream once sdUB is ready: its GEMM records the fork event
    if (side && !merged) fork_arm(ctx);
    auto sdub = [&] {
        GemmDesc g;
        g.prec = L->prec; g.a_src = bf ? SRC_BF16 : SRC_F32; g.b_src = bf ? SRC_BF16 : SRC_F32;
        g.A = L->dU; g.lda = out; g.B = L->Bt; g.ldb = out;
        g.M = N; g.N = r; g.K = out; g.alpha = L->s;
        if (bf) { g.Cb = static_cast<bf16*>(L->sdUB); g.ldcb = r; }
        else { g.C = static_cast<float*>(L->sdUB); g.ldc = r; }
        if (fold_btgb) {
            g.Mx = r; g.Ax = L->Ax; g.ldax = out; g.ldcx = r;
            if (bf) g.Cbx = static_cast<bf16*>(L->A2x);
            else g.Cx = static_cast<float*>(L->A2x);
        }
        gemm_run(ctx, g, scope(ctx, L, "lin_bwd_dub"));
    };
    if (!merged) sdub();
    // merged: sdUB = s dU B as r extra output columns of the dX GEMM (B rows from B^T) when they cost
    // it no extra round of workgroups; the dA partials then follow that GEMM
    // (with W_eff read as a [K][N] operand the extra columns read B itself, [out][r], as a [K][Nx]
    // operand: whole 64-column sub-tiles of dX's columns, in % 64 == 0)
    const bool sdub_cols = merged && dX && (L->Wmt || (in % 64 == 0 && r % 8 == 0)) && (ctx->rank_cols & 2) &&
                           gemm_extra_cols_free(ctx, N + (L->dora ? r : 0), in, out, r);
    // 4a. dA += sdUB^T X: the column-reduction partials only need sdUB and X, so they run before
    //     (on the second stream: beside) the dX GEMM; their sum is added to dA after the GEMM's
    //     extra dA rows (step 3), keeping the accumulation order of dA fixed. When the partials
    //     kernel sums them into dA itself (x_fused), the whole kernel runs after step 3.
    auto x_partials = [&] {
        if constexpr (sizeof(CT) == 2) {
            x_part = reduce_workspace(ctx, (size_t)x_S * 32 * in * sizeof(float));
            // the counters of the stream this runs on
            int* xc = nullptr;
            if (x_fused) {
                xc = tn_counters(ctx, ceil_div(in, TN_COLS), kFuseXSum);
                if (!xc) xc = stream_counters(ctx);
                SA3K_REQUIRE(xc != nullptr, "in-kernel reduction on a stream without counters");
            }
            const dim3 grid((unsigned)ceil_div(in, TN_COLS), (unsigned)x_S);
            KernelScope ks(ctx, scope(ctx, L, "lin_bwd_colred_x"), 2.0 * N * in * r);
            if (x_src == SRC_F32)
                launch_k(ctx, true, skinny_tn_kernel<TN_X, float>, grid, dim3(kThreads), 0, static_cast<const float*>(X),
                         static_cast<const bf16*>(L->sdUB), r, (const bf16*)nullptr, (const float*)nullptr,
                         (bf16*)nullptr, x_part, N, in, x_rows_per, dA, 1, xc, RowsArgs{}, (int64_t)in, (int64_t)r);
            else
                launch_k(ctx, true, skinny_tn_kernel<TN_X, bf16>, grid, dim3(kThreads), 0, static_cast<const bf16*>(X),
                         static_cast<const bf16*>(L->sdUB), r, (const bf16*)nullptr, (const float*)nullptr,
                         (bf16*)nullptr, x_part, N, in, x_rows_per, dA, 1, xc, RowsArgs{}, (int64_t)in, (int64_t)r);
            SA3K_LAUNCHED();
        } else {
            x_part = reduce_workspace(ctx, (size_t)x_S * R * in * sizeof(float));
            const dim3 grid((unsigned)ceil_div(in, kThreads), (unsigned)x_S);
            KernelScope ks(ctx, scope(ctx, L, "lin_bwd_colred_x"));
            if (x_src == SRC_F32)
                colred_x_kernel<float, CT, R><<<grid, kThreads, 0, ctx->stream>>>(
                    static_cast<const float*>(X), static_cast<const CT*>(L->sdUB), x_part, N, in, r, x_rows_per);
            else
                colred_x_kernel<bf16, CT, R><<<grid, kThreads, 0, ctx->stream>>>(
                    static_cast<const bf16*>(X), static_cast<const CT*>(L->sdUB), x_part, N, in, r, x_rows_per);
            SA3K_LAUNCHED();
        }
    };
    auto x_sum = [&] {
        if (x_fused) return;   // summed in-kernel
        KernelScope ks(ctx, scope(ctx, L, "lin_bwd_reduce"));
        const int64_t stride = (sizeof(CT) == 2 ? (int64_t)32 : (int64_t)R) * in;
        sum_splits_kernel<<<(unsigned)ceil_div((int64_t)r * in, kThreads), kThreads, 0, ctx->stream>>>(
            x_part, stride, x_S, (int64_t)r * in, dA, 1);
        SA3K_LAUNCHED();
    };
    if (!x_fused && !sdub_cols) {
        if (side) fork_fire(ctx);   // sdUB (merged: dU) and X are ready
        OnSide os(ctx, side);
        if (merged) sdub();
        x_partials();
    } else if (merged && !sdub_cols) {
        if (side) fork_fire(ctx);   // dU is ready
        OnSide os(ctx, side);
        sdub();
    }
    // 3. dX = dU W + sdUB A ; dora: dA += 2s B^T diag(gn) W + 2s^2 (B^T gn B) A as r extra rows
    //    of the same GEMM (they share the W^T tiles). Its last kernel records the next fork.
    if (side) fork_arm(ctx);
    // the B operand: W^T (stored layout or working copy) with the rank term as a second segment, or
    // W_eff^T when merged
    WOp wt = weight_operand(W, bf, true);
    // merged: W_eff^T, or W_eff itself read as a [K][N] operand when there is no transposed copy
    const int kn = merged && !L->Wmt ? 1 : 0;
    if (merged) wt = kn ? WOp{SRC_BF16, L->Wm, nullptr, in, 0} : WOp{SRC_BF16, L->Wmt, nullptr, out, 0};
    if (dX) {
        GemmDesc g;
        g.prec = L->prec; g.a_src = bf ? SRC_BF16 : SRC_F32; g.b_src = wt.src;
        g.A = L->dU; g.lda = out; g.B = wt.p; g.ldb = wt.ld; g.Bs = wt.s; g.ldbs = wt.lds; g.b_kn = kn;
        if (!merged) { g.A2 = L->sdUB; g.lda2 = r; g.B2 = L->At; g.ldb2 = r; g.K2 = r; }
        if (sdub_cols) {
            g.Nx = r; g.alpha_x = L->s; g.Cbn = static_cast<bf16*>(L->sdUB); g.ldcn = r;
            if (kn) { g.Bx = L->Bc; g.ldbx = r; }   // B [out][r]: K rows of r columns
            else { g.Bx = L->Bt; g.ldbx = out; }    // B^T [r][out]: r rows of K
        }
        g.M = N; g.N = in; g.K = out; g.alpha = 1.0f;
        g.C = dX; g.ldc = in; g.accumulate = dx_acc;
        if (epi) { g.ad = epi->ad; g.sb = epi->sb; g.bwd_done = epi->done; }
        if (L->dora) {
            g.Mx = r; g.Ax = L->Ax; g.ldax = out;
            if (!merged) { g.A2x = L->A2x; g.lda2x = r; }
            g.Cx = dA; g.ldcx = in; g.accumulate_x = 1;
        }
        gemm_run(ctx, g, scope(ctx, L, "lin_bwd_dx"));
    } else if (L->dora) {
        GemmDesc g;
        g.prec = L->prec; g.a_src = bf ? SRC_BF16 : SRC_F32; g.b_src = wt.src;
        g.A = L->Ax; g.lda = out; g.B = wt.p; g.ldb = wt.ld; g.Bs = wt.s; g.ldbs = wt.lds; g.b_kn = kn;
        if (!merged) { g.A2 = L->A2x; g.lda2 = r; g.B2 = L->At; g.ldb2 = r; g.K2 = r; }
        g.M = r; g.N = in; g.K = out; g.alpha = 1.0f;
        g.C = dA; g.ldc = in; g.accumulate = 1;
        gemm_run(ctx, g, scope(ctx, L, "lin_bwd_dora_da"));
    }
    // 4b. the partial sums into dA, after step 3
    if (side) fork_fire(ctx);   // the dX GEMM has added its dA rows (and written sdUB)
    {
        OnSide os(ctx, side);
        if (x_fused || sdub_cols) x_partials();
        x_sum();
    }
    if (side) side_join_unless_deferred(ctx);
}

// ---------------------------------------------------------------- grouped adapter refresh
// One descriptor per member linear; every stage is one launch over the whole group. The grids are
// compact: block_member[b] names the member a block works for and the member's first block of the
// stage sits in PrepDesc::blk0[stage], so no block is launched for a member that has no work there
// (a grid sized for the largest member times the member count launches hundreds of thousands of
// empty blocks).
enum PrepStage { kStageConvert = 0, kStagePt = 1, kStageGram = 2, kStageTerms = 3, kStageMerge = 4, kStages = 5 };
constexpr int kPtRows = 256;                  // rows of P^T per block (4 waves x 64)

constexpr int kTermRows = 64;                 // DoRA rows per block (8 passes of 8)

struct PrepDesc {
    const float *A, *B, *mag, *bnsq;   // adapter (device) [r][in], [out][r], [out], [out]
    void *Ac, *At, *Bc, *Bt;           // compute-type copies [r][in], [in][r], [out][r], [r][out]
                                       // (bf16, or f32 in a group of f32-precision linears)
    const bf16* W;                     // bf16 working copy of the base [out][in]
    float *Pt, *G, *BG, *nsq, *d;
    int in, out;
    int blk0[kStages];                 // first block of this member in each stage's grid
    // merged mode: the stored base (element type wtype; Q8_0: quants in Wsrc, f16 scales in Wsc)
    // and the bf16 W_eff = W + s B A in both layouts
    const void* Wsrc;
    const void* Wsc;
    int wtype;
    bf16 *Wm, *Wmt;
};

// Ac/At/Bc/Bt from A and B. A block converts one 64-wide tile: columns [64t, 64t + 64) of A
// (all r rows) for its first ceil(in/64) blocks, then rows [64t, 64t + 64) of B (all r columns).
// The copies in the source layout are written as read; the transposed copies go through LDS so
// every store is a contiguous row (a direct transposed store touches one cache segment per value).
template <class CT>
__global__ __launch_bounds__(kThreads) void group_convert_kernel(const PrepDesc* __restrict__ ds,
                                                                 const int* __restrict__ block_member, int r) {
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    __shared__ CT tile[64][34];   // [tile index][rank], padded
    CT* const Ac = static_cast<CT*>(q.Ac);
    CT* const At = static_cast<CT*>(q.At);
    CT* const Bc = static_cast<CT*>(q.Bc);
    CT* const Bt = static_cast<CT*>(q.Bt);
    const int t = blockIdx.x - q.blk0[kStageConvert];
    const int a_tiles = (q.in + 63) / 64;
    const bool is_a = t < a_tiles;
    const int64_t base = (int64_t)(is_a ? t : t - a_tiles) * 64;
    const int64_t extent = is_a ? q.in : q.out;
    // load: element (rank a, index base + j); A is [r][in] (index along a row), B is [out][r]
    for (int e = threadIdx.x; e < 64 * 32; e += kThreads) {
        int a, j;
        if (is_a) { a = e / 64; j = e % 64; }   // consecutive threads: consecutive columns of row a
        else { j = e / 32; a = e % 32; }        // consecutive threads: consecutive ranks of row j
        const int64_t idx = base + j;
        if (a >= r || idx >= extent) continue;
        const float v = is_a ? q.A[(int64_t)a * q.in + idx] : q.B[idx * r + a];
        const CT b = (CT)v;
        tile[j][a] = b;
        if (is_a) Ac[(int64_t)a * q.in + idx] = b;
        else Bc[idx * r + a] = b;
    }
    __syncthreads();
    // transposed stores: At [in][r] (rows of r ranks), Bt [r][out] (rows of 64 indices)
    for (int e = threadIdx.x; e < 64 * 32; e += kThreads) {
        int a, j;
        if (is_a) { j = e / 32; a = e % 32; }
        else { a = e / 64; j = e % 64; }
        const int64_t idx = base + j;
        if (a >= r || idx >= extent) continue;
        if (is_a) At[idx * r + a] = tile[j][a];
        else Bt[(int64_t)a * q.out + idx] = tile[j][a];
    }
}

// P^T[a][o] = sum_i A[a][i] W[o][i] for every member, v_mfma_f32_16x16x32_bf16: one block per 256
// rows o of one member, each wave 64 rows (4 row blocks of 16) x 32 ranks, so a fragment of A
// serves 4 MFMAs (A is read from L2 once per 64 rows of W, not per 16). Both operands come straight
// from global memory (a lane's 8 consecutive K elements are 16 contiguous bytes of a row). The K
// loop runs over 64-wide chunks with two register sets: the next chunk's loads are issued before
// the current chunk's MFMAs; the loads are unconditional (rows and chunks clamped into range), so
// the wait before each chunk counts only the other set's loads.
template <bool HI>   // HI: the rank exceeds 16, so a second 16-rank block of P^T rows exists
__global__ __launch_bounds__(kThreads) void group_pt_kernel(const PrepDesc* __restrict__ ds,
                                                            const int* __restrict__ block_member, int r) {
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, g = lane >> 4;
    const int64_t o0 = (int64_t)(blockIdx.x - q.blk0[kStagePt]) * kPtRows + wave * 64;
    if (o0 >= q.out) return;   // wave-uniform
    constexpr int WR = 4;
    // buffer loads: the member's W and Ac in two descriptors (extents checked on the host to fit
    // 31 bits), a loop-invariant 32-bit byte offset per lane and row, the chunk's K in the scalar
    // offset; the last rows are clamped to the last valid row (their results are not stored)
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(q.W), (short)0, (int)((int64_t)q.out * q.in * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(q.Ac, (short)0, (int)((int64_t)r * q.in * 2), 0x00020000);
    uint32_t wof[WR];
#pragma unroll
    for (int j = 0; j < WR; ++j) wof[j] = (uint32_t)((std::min<int64_t>(o0 + 16 * j + r16, q.out - 1) * q.in + 8 * g) * 2);
    const uint32_t a0of = (uint32_t)(((int64_t)min(r16, r - 1) * q.in + 8 * g) * 2);
    const uint32_t a1of = (uint32_t)(((int64_t)min(16 + r16, r - 1) * q.in + 8 * g) * 2);
    struct Set {
        bf16x8 w[2][WR], a0[2], a1[2];
    };
    auto ld16 = [](__amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t so) {
        return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, (int)so, 0));
    };
    auto load = [&](Set& S, int c) {   // chunk c: K [64c, 64c + 64), two K32 steps
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const uint32_t ko = (uint32_t)(c * 64 + 32 * st) * 2;   // wave-uniform
#pragma unroll
            for (int j = 0; j < WR; ++j) S.w[st][j] = ld16(rw, wof[j], ko);
            S.a0[st] = ld16(ra, a0of, ko);
            if (HI) S.a1[st] = ld16(ra, a1of, ko);
        }
    };
    f32x4 acc[WR][2];
#pragma unroll
    for (int j = 0; j < WR; ++j) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const Set& S) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int j = 0; j < WR; ++j) {
                acc[j][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(S.w[st][j], S.a0[st], acc[j][0], 0, 0, 0);
                if (HI) acc[j][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(S.w[st][j], S.a1[st], acc[j][1], 0, 0, 0);
            }
    };
    const int nc = q.in / 64;
    Set sa, sb;
    int c = 0;
    if (nc & 1) {   // an odd chunk first, so the pipelined loop below runs whole pairs
        load(sa, 0);
        mma(sa);
        c = 1;
    }
    load(sa, c);
    // the scheduling barriers keep each set's loads ahead of the other set's products (the compiler
    // would otherwise sink them to their first use and serialize load and MFMA)
    for (; c < nc; c += 2) {
        load(sb, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(sa);
        __builtin_amdgcn_sched_barrier(0);
        load(sa, min(c + 2, nc - 1));   // past the last pair: a discarded reload of the last chunk
        __builtin_amdgcn_sched_barrier(0);
        mma(sb);
        __builtin_amdgcn_sched_barrier(0);
    }
    // D[i][j]: o = o0 + 16 jr + 4g + v, rank = r16 (+16)
#pragma unroll
    for (int j = 0; j < WR; ++j) {
        const int64_t o = o0 + 16 * j + 4 * g;
        if (o >= q.out) continue;   // out is a multiple of 16: whole 4-row groups
        if (r16 < r)
            *reinterpret_cast<float4*>(q.Pt + (int64_t)r16 * q.out + o) =
                make_float4(acc[j][0][0], acc[j][0][1], acc[j][0][2], acc[j][0][3]);
        if (HI && 16 + r16 < r)
            *reinterpret_cast<float4*>(q.Pt + (int64_t)(16 + r16) * q.out + o) =
                make_float4(acc[j][1][0], acc[j][1][1], acc[j][1][2], acc[j][1][3]);
    }
}

// G = A A^T in double, two launches. Pass 1: one block per 256 columns of one member forms the
// r x r partial sum over its columns (A's 32 x 256 slice staged in LDS; each thread owns 4 entries
// (a, b) and adds the columns in order). Pass 2: one block per member sums its partials in column
// order. Deterministic; each entry is a double sum rounded once to float.
constexpr int kGramCols = 256;
__global__ __launch_bounds__(kThreads) void group_gram_part_kernel(const PrepDesc* __restrict__ ds,
                                                                   const int* __restrict__ block_member, int r,
                                                                   double* __restrict__ part) {
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    const int c = blockIdx.x - q.blk0[kStageGram];
    __shared__ float sa[32][kGramCols + 1];
    const int64_t k0 = (int64_t)c * kGramCols;
    const int kn = (int)std::min<int64_t>(kGramCols, q.in - k0);
    for (int e = threadIdx.x; e < 32 * kGramCols; e += kThreads) {
        const int a = e / kGramCols, k = e % kGramCols;
        sa[a][k] = (a < r && k < kn) ? q.A[(int64_t)a * q.in + k0 + k] : 0.f;
    }
    __syncthreads();
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    const int a = threadIdx.x / 8, b0 = (threadIdx.x % 8) * 4;   // entries (a, b0..b0+3)
    for (int k = 0; k < kn; ++k) {
        const double x = sa[a][k];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += x * (double)sa[b0 + j][k];
    }
    double* out = part + (int64_t)blockIdx.x * 1024;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[a * 32 + b0 + j] = acc[j];
}

__global__ __launch_bounds__(kThreads) void group_gram_sum_kernel(const PrepDesc* __restrict__ ds, int r,
                                                                  const double* __restrict__ part) {
    const PrepDesc& q = ds[blockIdx.x];
    const int chunks = (q.in + kGramCols - 1) / kGramCols;
    for (int e = threadIdx.x; e < 32 * 32; e += kThreads) {
        const int a = e / 32, b = e % 32;
        if (a >= r || b >= r) continue;
        double sum = 0.0;
        for (int c = 0; c < chunks; ++c) sum += part[(int64_t)(q.blk0[kStageGram] + c) * 1024 + e];
        q.G[a * r + b] = (float)sum;
    }
}

// P^T[a][o] = sum_i A[a][i] W[o][i] in f32 for the members of an f32-precision group (the DiT's
// head / tail linears), from the stored base (f32 or f16, decoded exactly to f32): one block per
// kPtRowsF32 = 64 rows o of one member, the K loop in 64-wide chunks staged in LDS (W rows as f32,
// A's r x 64 slice); wave w owns ranks 8w..8w+7 of all 64 rows, lane l row l, so the A reads are
// wave-uniform broadcasts and the W reads fall into distinct banks (row pitch 65). Each sum runs
// over i in order: deterministic. The input dimension is a multiple of 64 (checked on the host).
constexpr int kPtRowsF32 = 64;
template <int WT>
__global__ __launch_bounds__(kThreads) void group_pt_f32_kernel(const PrepDesc* __restrict__ ds,
                                                                const int* __restrict__ block_member, int r) {
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    if (q.wtype != WT) return;   // another launch serves this member's element type
    __shared__ float ws[kPtRowsF32][65];
    __shared__ float as[32][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t o0 = (int64_t)(blockIdx.x - q.blk0[kStagePt]) * kPtRowsF32;
    const int in = q.in;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int k0 = 0; k0 < in; k0 += 64) {
        // W rows o0 .. o0 + 63, columns k0 .. k0 + 63: 16 columns per thread (rows past out: zeros)
        {
            const int row = tid >> 2, c0 = (tid & 3) * 16;
            const int64_t o = o0 + row;
            float v[16];
            if (o < q.out) {
                if (WT == SA3K_TYPE_F32) {
                    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(q.Wsrc) + o * in + k0 + c0);
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float4 f = src[u];
                        v[4 * u] = f.x; v[4 * u + 1] = f.y; v[4 * u + 2] = f.z; v[4 * u + 3] = f.w;
                    }
                } else {
                    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(q.Wsrc) + o * in + k0 + c0);
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint4 h = src[u];
                        const uint32_t w4[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[8 * u + 2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w4[e] & 0xffffu));
                            v[8 * u + 2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w4[e] >> 16));
                        }
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) ws[row][c0 + e] = v[e];
        }
        // A[:, k0 .. k0 + 63]: 8 columns per thread (ranks past r: zeros)
        {
            const int a = tid >> 3, c0 = (tid & 7) * 8;
            const float* A = static_cast<const float*>(q.A);
#pragma unroll
            for (int e = 0; e < 8; ++e) as[a][c0 + e] = a < r ? A[(int64_t)a * in + k0 + c0 + e] : 0.f;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < 64; ++k) {
            const float w = ws[lane][k];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += w * as[8 * wave + j][k];
        }
        __syncthreads();
    }
    const int64_t o = o0 + lane;
    if (o >= q.out) return;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (8 * wave + j < r) q.Pt[(int64_t)(8 * wave + j) * q.out + o] = acc[j];
}

// nsq, d and BG = B G for kTermRows rows of one member per block (G staged in LDS once per block)
__global__ __launch_bounds__(kThreads) void group_dora_terms_kernel(const PrepDesc* __restrict__ ds,
                                                                    const int* __restrict__ block_member, int r,
                                                                    float s) {
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    __shared__ float gs[32][33];
    __shared__ float bs[8][32];
    const int ol = threadIdx.x >> 5, a = threadIdx.x & 31;
    const int64_t row0 = (int64_t)(blockIdx.x - q.blk0[kStageTerms]) * kTermRows;
    for (int k = threadIdx.x; k < 32 * 32; k += kThreads) {
        const int i = k >> 5, j = k & 31;
        gs[i][j] = (i < r && j < r) ? q.G[i * r + j] : 0.f;
    }
    for (int pass = 0; pass < kTermRows / 8; ++pass) {
        const int64_t o = row0 + pass * 8 + ol;
        __syncthreads();   // G staged; the previous pass is done with bs
        bs[ol][a] = (o < q.out && a < r) ? q.B[o * r + a] : 0.f;
        __syncthreads();
        float gv = 0.f;
#pragma unroll 8
        for (int c = 0; c < 32; ++c) gv += bs[ol][c] * gs[c][a];
        float t2 = 0.f, t3 = 0.f;
        if (o < q.out && a < r) {
            q.BG[o * r + a] = gv;
            t2 = q.Pt[(int64_t)a * q.out + o] * bs[ol][a];
            t3 = bs[ol][a] * gv;
        }
        for (int off = 16; off > 0; off >>= 1) {
            t2 += __shfl_xor(t2, off, 32);
            t3 += __shfl_xor(t3, off, 32);
        }
        if (a == 0 && o < q.out) {
            const float n2 = q.bnsq[o] + 2.0f * s * t2 + s * s * t3;
            q.nsq[o] = n2;
            q.d[o] = q.mag[o] / sqrtf(n2);
        }
    }
}


// ---- merged refresh: W_eff = W + s B A, once per optimizer step
// One block per 64 output rows of one member walks the member's input dimension in 64-wide chunks:
//   * the stored base chunk (f32 / f16 / bf16, or Q8_0 quants times their f16 scale: the exact
//     decoded value) is staged in LDS as f32, the next chunk's raw bytes already in flight;
//   * delta = B A on v_mfma_f32_16x16x32_bf16 (each wave 16 rows x 64 columns, the rank as K),
//     W_eff = W + s delta rounded once to bf16 and staged in LDS in both layouts, from which every
//     thread stores 32 contiguous bytes of a row of W_eff [out][in] and of W_eff^T [in][out];
//   * dora: nsq = bnsq + sum_i (2 W s delta + (s delta)^2) in double (the expansion of
//     |W + s B A|^2 - |W|^2, so no cancellation against bnsq), and P = W_eff A^T on MFMA from the
//     bf16 W_eff rows, which the backward's dB term 2 s gn P and the magnitude d = m / sqrt(nsq)
//     need. The row sums are reduced in a fixed lane order: deterministic.
constexpr int kMergeRows = 64;
constexpr int kMergeEP = 72;   // bf16 row pitch of the staged W_eff chunks (144 bytes: 16-byte aligned rows)

// stored element type of a merge launch: its raw bytes per element and its decode
template <int TYPE>
struct MergeType;
template <>
struct MergeType<SA3K_TYPE_F32> {
    static constexpr int kBytes = 4;
    __device__ static float get(const char* row, int k, float) { return reinterpret_cast<const float*>(row)[k]; }
};
template <>
struct MergeType<SA3K_TYPE_F16> {
    static constexpr int kBytes = 2;
    __device__ static float get(const char* row, int k, float) {
        return (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t*>(row)[k]);
    }
};
template <>
struct MergeType<SA3K_TYPE_BF16> {
    static constexpr int kBytes = 2;
    __device__ static float get(const char* row, int k, float) {
        return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(row)[k] << 16);
    }
};
template <>
struct MergeType<SA3K_TYPE_Q8_0> {   // quants; the f16 block scale is passed in (exact decode d * q)
    static constexpr int kBytes = 1;
    __device__ static float get(const char* row, int k, float sc) { return (float)reinterpret_cast<const int8_t*>(row)[k] * sc; }
};

// 16-byte global-memory load (address space 1: counted by vmcnt only, unlike a flat access)
typedef unsigned u32x4g __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4g g_cu4;
__device__ __forceinline__ uint4 ldg16(const void* p) {
    const u32x4g v = *(g_cu4*)p;
    return uint4{v.x, v.y, v.z, v.w};
}

// Every chunk's operands (the raw base chunk, the 64 rows of A^T and the r x 64 slice of A) are
// loaded cooperatively one chunk ahead, all before the current chunk's stores: the wait for them at
// the next chunk then does not include those stores (vmcnt counts loads and stores in issue order).
template <int TYPE>
__global__ __launch_bounds__(kThreads) void group_merge_kernel(const PrepDesc* __restrict__ ds,
                                                               const int* __restrict__ block_member, int r, float s) {
    using MT = MergeType<TYPE>;
    constexpr int RB = 64 * MT::kBytes;                    // raw bytes of one chunk row
    constexpr int RP = RB + 16;                             // LDS pitch of the raw chunk rows
    constexpr int NQ = RB * kMergeRows / 16 / kThreads;     // 16-byte raw loads per thread per chunk (1, 2 or 4)
    constexpr int TPR = RB / 16;                            // threads per raw chunk row
    constexpr int AP = 80;                                  // LDS pitch of the A^T rows (64 bytes + 16)
    constexpr int CP = 144;                                 // LDS pitch of the A rows (128 bytes + 16)
    const PrepDesc& q = ds[block_member[blockIdx.x]];
    if (q.wtype != TYPE) return;   // a member of another element type (its own launch)
    __shared__ __attribute__((aligned(16))) char wraw[kMergeRows * RP];
    __shared__ __attribute__((aligned(16))) char ats[64 * AP];                  // A^T rows of the chunk [i][a]
    __shared__ __attribute__((aligned(16))) char acs[32 * CP];                  // A rows of the chunk [a][i]
    __shared__ __attribute__((aligned(16))) float wsc[kMergeRows][2];           // Q8_0 scales of the chunk
    __shared__ __attribute__((aligned(16))) bf16 et[kMergeRows][kMergeEP];      // W_eff [o][i] of the chunk
    __shared__ __attribute__((aligned(16))) bf16 ett[kMergeRows][kMergeEP];     // W_eff^T [i][o] of the chunk
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g = lane >> 4;
    const int64_t in = q.in, out = q.out;
    const int64_t o0 = (int64_t)(blockIdx.x - q.blk0[kStageMerge]) * kMergeRows;
    const bool dora = q.mag != nullptr;
    const bool hi = r > 16;
    const char* wsrc = static_cast<const char*>(q.Wsrc);
    // this thread's slice of the A^T rows (row tid / 4, bytes 16 (tid % 4)) and of the A rows
    // (row tid / 8, bytes 16 (tid % 8)); slices past the rank read a valid address and are zeroed
    const int at_row = tid >> 2, at_b = 16 * (tid & 3), ac_row = tid >> 3, ac_b = 16 * (tid & 7);
    const bool at_ok = at_b < 2 * r, ac_ok = ac_row < r;
    const char* at_src = reinterpret_cast<const char*>(q.At) + (int64_t)at_row * r * 2 + (at_ok ? at_b : 0);
    const char* ac_src = reinterpret_cast<const char*>(q.Ac) + (int64_t)(ac_ok ? ac_row : 0) * in * 2 + ac_b;
    struct Stage {
        uint4 w[NQ], at, ac;
        uint32_t sc;   // Q8_0: the chunk row's two f16 block scales (threads < 64)
    } st;
    auto load = [&](int64_t i0) {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int e = tid + k * kThreads, row = e / TPR;
            const int64_t o = min(o0 + row, out - 1);   // rows past out are never stored
            st.w[k] = ldg16(wsrc + (o * in + i0) * MT::kBytes + (e % TPR) * 16);
        }
        st.at = ldg16(at_src + i0 * r * 2);
        st.ac = ldg16(ac_src + i0 * 2);
        if constexpr (TYPE == SA3K_TYPE_Q8_0) {
            const int64_t o = min(o0 + (tid & 63), out - 1);
            st.sc = *(__attribute__((address_space(1))) const uint32_t*)(static_cast<const uint16_t*>(q.Wsc) + o * (in / 32) + i0 / 32);
        }
    };
    // delta's A operand: the rank entries 8g.. of B row o (this wave's 16 rows), loop-invariant
    const int64_t ob = min(o0 + 16 * wave + l16, out - 1);
    const bf16x8 zero8 = {};
    const bf16x8 bop = 8 * g < r ? __builtin_bit_cast(bf16x8, ldg16(static_cast<const bf16*>(q.Bc) + ob * r + (8 * g < r ? 8 * g : 0))) : zero8;
    double nacc[4] = {0.0, 0.0, 0.0, 0.0};   // rows 16 wave + 4g + v, this lane's columns
    f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = {0.f, 0.f, 0.f, 0.f};
    const uint32_t wbytes = (uint32_t)(out * in * 2);   // < 2^31 (checked when the group is built)
    const __amdgpu_buffer_rsrc_t rs_m = __builtin_amdgcn_make_buffer_rsrc(q.Wm, (short)0, (int)wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs_mt = __builtin_amdgcn_make_buffer_rsrc(q.Wmt, (short)0, (int)wbytes, 0x00020000);
    load(0);
    // the first chunk landed: the loop head's wait then only reflects the loop body's issue order
    // (a scheduler-reordered prologue would otherwise force a full wait there every chunk)
    __builtin_amdgcn_s_waitcnt(0x3F70);   // vmcnt(0)
    const int nc = (int)(in / 64);
    for (int c = 0; c < nc; ++c) {
        const int64_t i0 = (int64_t)c * 64;
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int e = tid + k * kThreads;
            *reinterpret_cast<uint4*>(wraw + (e / TPR) * RP + (e % TPR) * 16) = st.w[k];
        }
        {   // slices past the rank are zeroed arithmetically (no branch: see the stores below)
            const uint32_t ma = at_ok ? ~0u : 0u, mc = ac_ok ? ~0u : 0u;
            *reinterpret_cast<uint4*>(ats + at_row * AP + at_b) = uint4{st.at.x & ma, st.at.y & ma, st.at.z & ma, st.at.w & ma};
            *reinterpret_cast<uint4*>(acs + ac_row * CP + ac_b) = uint4{st.ac.x & mc, st.ac.y & mc, st.ac.z & mc, st.ac.w & mc};
        }
        if constexpr (TYPE == SA3K_TYPE_Q8_0) {
            if (tid < kMergeRows) {
                wsc[tid][0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(st.sc & 0xffffu));
                wsc[tid][1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(st.sc >> 16));
            }
        }
        if (c + 1 < nc) load(i0 + 64);   // the next chunk in flight
        __syncthreads();   // the chunk is staged; the previous chunk's W_eff tiles are consumed
        // The P product's A operands (this chunk's A rows) are read before the second barrier: a
        // wave past that barrier may already be writing the next chunk's A rows into acs.
        bf16x8 pa[2][2] = {};
        if (dora) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                pa[ks][0] = *reinterpret_cast<const bf16x8*>(acs + l16 * CP + (32 * ks + 8 * g) * 2);
                if (hi) pa[ks][1] = *reinterpret_cast<const bf16x8*>(acs + (16 + l16) * CP + (32 * ks + 8 * g) * 2);
            }
        }
        // W_eff at (row 16 wave + 4g + v, column 16j + l16)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 atj = *reinterpret_cast<const bf16x8*>(ats + (16 * j + l16) * AP + 16 * g);
            const f32x4 dl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bop, atj, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            bf16 e4[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = 16 * wave + 4 * g + v, col = 16 * j + l16;
                const float sc = TYPE == SA3K_TYPE_Q8_0 ? wsc[row][col / 32] : 0.f;
                const float w = MT::get(wraw + row * RP, col, sc);
                const float sd = s * dl[v];
                const bf16 e = (bf16)(w + sd);
                e4[v] = e;
                et[row][col] = e;
                if (dora) nacc[v] += (double)sd * (2.0 * (double)w + (double)sd);
            }
            if (q.Wmt) *reinterpret_cast<uint2*>(&ett[16 * j + l16][16 * wave + 4 * g]) = __builtin_bit_cast(uint2, e4);
        }
        __syncthreads();   // et, ett staged
        if (dora) {   // P += W_eff A^T over the chunk (rows 16 wave + l16 of W_eff as the A operand)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const bf16x8 wa = *reinterpret_cast<const bf16x8*>(&et[16 * wave + l16][32 * ks + 8 * g]);
                p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, pa[ks][0], p0, 0, 0, 0);
                if (hi) p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, pa[ks][1], p1, 0, 0, 0);
            }
        }
        {   // 32 contiguous bytes of a W_eff row and of a W_eff^T row per thread, after every load.
            // Buffer stores: rows past out get an offset beyond the extent, which the hardware drops,
            // so no branch makes the wait for the next chunk's loads also wait for these stores.
            const int lr = tid >> 2, lc = 16 * (tid & 3);
            const uint4* fr = reinterpret_cast<const uint4*>(&et[lr][lc]);
            const uint4* tr = reinterpret_cast<const uint4*>(&ett[lr][lc]);
            const uint32_t fo = o0 + lr < out ? (uint32_t)(((o0 + lr) * in + i0 + lc) * 2) : 0xFFFFFFE0u;
            const uint32_t to = o0 + lc < out ? (uint32_t)(((i0 + lr) * out + o0 + lc) * 2) : 0xFFFFFFE0u;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4g, fr[0]), rs_m, fo, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4g, fr[1]), rs_m, fo + 16, 0, 0);
            if (q.Wmt) {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4g, tr[0]), rs_mt, to, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4g, tr[1]), rs_mt, to + 16, 0, 0);
            }
        }
    }
    if (!dora) return;
    // row sums over the 16 lanes of a group (fixed butterfly order), then nsq, d and P^T
#pragma unroll
    for (int v = 0; v < 4; ++v)
        for (int off = 1; off < 16; off <<= 1) nacc[v] += __shfl_xor(nacc[v], off, 16);
    const int64_t orow = o0 + 16 * wave + 4 * g;
    if (orow >= out) return;   // out is a multiple of 16: a 4-row group is wholly in or out
    if (l16 == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float n2 = (float)((double)q.bnsq[orow + v] + nacc[v]);
            q.nsq[orow + v] = n2;
            q.d[orow + v] = q.mag[orow + v] / sqrtf(n2);
        }
    }
    if (l16 < r) *reinterpret_cast<float4*>(q.Pt + (int64_t)l16 * out + orow) = make_float4(p0[0], p0[1], p0[2], p0[3]);
    if (hi && 16 + l16 < r)
        *reinterpret_cast<float4*>(q.Pt + (int64_t)(16 + l16) * out + orow) = make_float4(p1[0], p1[1], p1[2], p1[3]);
}

}  // namespace

namespace sa3k {

void lin_set_tag(sa3k_lin* l, const char* tag) { l->tag = tag; }

bf16* lin_du(sa3k_lin* L) { return static_cast<bf16*>(L->dU); }

const float* lin_du_scale(const sa3k_lin* L) { return L->rank > 0 && L->dora ? L->d : nullptr; }

void lin_backward_du(sa3k_ctx* ctx, sa3k_lin* L, int x_type, const void* X, int64_t N, float* dX, int dx_accumulate,
                     float* dA, float* dB, float* dm, const DxEpi* epi) {
    SA3K_REQUIRE(L && X, "null pointer");
    SA3K_REQUIRE(L->prec == SA3K_PREC_BF16, "a precomputed dU needs a bf16-precision linear");
    SA3K_REQUIRE(N == L->saved_tokens, "backward must follow a forward over the same tokens");
    SA3K_REQUIRE(L->rank == 0 || (dA && dB), "adapter gradients need dA/dB buffers");
    SA3K_REQUIRE(!L->dora || dm, "dora needs a magnitude gradient buffer");
    SA3K_REQUIRE(x_type == SA3K_TYPE_F32 || x_type == SA3K_TYPE_BF16, "activation type must be f32 or bf16");
    const int xs = x_type == SA3K_TYPE_F32 ? SRC_F32 : SRC_BF16;
    if (L->rank <= 16) lin_backward_t<bf16, 16>(ctx, L, xs, X, N, nullptr, dX, dx_accumulate, dA, dB, dm, epi);
    else lin_backward_t<bf16, 32>(ctx, L, xs, X, N, nullptr, dX, dx_accumulate, dA, dB, dm, epi);
}

void weight_fwd_operand(const sa3k_weight* W, GemmDesc& g) {
    const WOp wo = weight_operand(W, g.prec == SA3K_PREC_BF16, false);
    g.b_src = wo.src;
    g.B = wo.p;
    g.ldb = wo.ld;
    g.Bs = wo.s;
    g.ldbs = wo.lds;
}

struct LinGroup {
    std::vector<sa3k_lin*> lins;
    std::vector<const float*> B, mag;
    PrepDesc* dev = nullptr;
    int* block_member[kStages] = {};   // per stage: the member of every block
    int blocks[kStages] = {};
    int n = 0, r = 0, dora = 0, merged = 0;
    int f32 = 0;   // members compute in f32: f32 copies, P on the VALU from the stored base
    float s = 1.0f;
};

void lin_group_free(LinGroup* g) {
    if (!g) return;
    if (g->dev) (void)hipFree(g->dev);
    for (int* b : g->block_member)
        if (b) (void)hipFree(b);
    delete g;
}

LinGroup* lin_group_create(sa3k_ctx* ctx, sa3k_lin* const* lins, int n, const float* const* A, const float* const* B,
                           const float* const* mag, const float* const* bnsq, float scale, int dora) {
    SA3K_REQUIRE(n > 0 && lins && A && B && (!dora || (mag && bnsq)), "bad linear group");
    LinGroup* g = new LinGroup();
    try {
        g->n = n;
        g->r = lins[0]->rank;
        g->dora = dora ? 1 : 0;
        g->s = scale;
        // f32-precision members: the two-segment refresh with f32 copies and an f32 P
        g->f32 = lins[0]->prec == SA3K_PREC_F32 ? 1 : 0;
        g->merged = ctx->lin_merge && !g->f32 ? 1 : 0;
        std::vector<PrepDesc> h(n);
        std::vector<int> bm[kStages];
        for (int i = 0; i < n; ++i) {
            sa3k_lin* L = lins[i];
            SA3K_REQUIRE(L->prec == lins[0]->prec && L->rank == g->r && g->r > 0,
                         "a linear group needs linears of one precision and rank");
            if (g->f32)
                SA3K_REQUIRE((L->W->type == SA3K_TYPE_F32 || L->W->type == SA3K_TYPE_F16) && L->W->in % 64 == 0,
                             "an f32 linear group needs f32 / f16 bases with inputs a multiple of 64");
            else
                SA3K_REQUIRE(L->prec == SA3K_PREC_BF16 && (g->merged || L->W->wb),
                             "a bf16 linear group needs bf16 working copies unless merged");
            SA3K_REQUIRE(A[i] && B[i] && (!dora || (mag[i] && bnsq[i])), "missing adapter pointer");
            const int64_t in = L->W->in, out = L->W->out;
            SA3K_REQUIRE(out % 64 == 0 || out % 16 == 0, "group output dimension must be a multiple of 16");
            SA3K_REQUIRE((int64_t)out * in * 2 < ((int64_t)1 << 31), "group member weight above 2 GiB");
            PrepDesc& q = h[i];
            q.A = A[i]; q.B = B[i]; q.mag = dora ? mag[i] : nullptr; q.bnsq = dora ? bnsq[i] : nullptr;
            q.Ac = L->Ac; q.At = L->At; q.Bc = L->Bc; q.Bt = L->Bt;
            q.W = static_cast<const bf16*>(L->W->wb);
            q.Pt = L->Pt; q.G = L->G; q.BG = L->BG; q.nsq = L->nsq; q.d = L->d;
            q.in = (int)in; q.out = (int)out;
            q.Wsrc = L->W->w; q.Wsc = L->W->ws; q.wtype = L->W->type;
            q.Wm = q.Wmt = nullptr;
            if (g->merged) {
                // the dX product reads W_eff as it lies ([out][in] as a [K][N] operand) unless the
                // transposed copy is asked for (option merge_kn 0)
                if (!L->Wm) L->Wm = dev_alloc<bf16>(in * out);
                if (!ctx->merge_kn && !L->Wmt) L->Wmt = dev_alloc<bf16>(in * out);
                if (ctx->merge_kn && L->Wmt) {
                    SA3K_HIP(hipFree(L->Wmt));
                    L->Wmt = nullptr;
                }
                q.Wm = static_cast<bf16*>(L->Wm);
                q.Wmt = static_cast<bf16*>(L->Wmt);
            }
            const int64_t per_stage[kStages] = {ceil_div(in, 64) + ceil_div(out, 64),
                                                ceil_div(out, g->f32 ? kPtRowsF32 : kPtRows),
                                                ceil_div(in, kGramCols), ceil_div(out, kTermRows),
                                                ceil_div(out, kMergeRows)};
            for (int st = 0; st < kStages; ++st) {
                if (st == kStageMerge) continue;
                q.blk0[st] = (int)bm[st].size();
                bm[st].insert(bm[st].end(), (size_t)per_stage[st], i);
            }
            g->lins.push_back(L);
            g->B.push_back(B[i]);
            g->mag.push_back(dora ? mag[i] : nullptr);
        }
        {   // merge blocks walk a member's whole input dimension: the longest members go first
            std::vector<int> order(n);
            for (int i = 0; i < n; ++i) order[i] = i;
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return h[a].in > h[b].in; });
            for (int i : order) {
                h[i].blk0[kStageMerge] = (int)bm[kStageMerge].size();
                bm[kStageMerge].insert(bm[kStageMerge].end(), (size_t)ceil_div(h[i].out, kMergeRows), i);
            }
        }
        SA3K_HIP(hipMalloc(&g->dev, sizeof(PrepDesc) * n));
        SA3K_HIP(hipMemcpyAsync(g->dev, h.data(), sizeof(PrepDesc) * n, hipMemcpyHostToDevice, ctx->stream));
        sa3k_note_main(ctx);
        for (int st = 0; st < kStages; ++st) {
            g->blocks[st] = (int)bm[st].size();
            if (bm[st].empty()) continue;
            SA3K_HIP(hipMalloc(&g->block_member[st], sizeof(int) * bm[st].size()));
            SA3K_HIP(hipMemcpyAsync(g->block_member[st], bm[st].data(), sizeof(int) * bm[st].size(),
                                    hipMemcpyHostToDevice, ctx->stream));
            sa3k_note_main(ctx);
        }
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    } catch (...) {
        lin_group_free(g);
        throw;
    }
    return g;
}

void lin_group_prepare(sa3k_ctx* ctx, LinGroup* g) {
    for (int i = 0; i < g->n; ++i) {   // the per-linear state sa3k_lin_prepare sets
        sa3k_lin* L = g->lins[i];
        L->s = g->s;
        L->dora = g->dora;
        L->B = g->B[i];
        L->mag = g->mag[i];
        L->merged = g->merged;
    }
    {
        KernelScope ks(ctx, "group_convert");
        auto* kern = g->f32 ? group_convert_kernel<float> : group_convert_kernel<bf16>;
        kern<<<(unsigned)g->blocks[kStageConvert], kThreads, 0, ctx->stream>>>(g->dev, g->block_member[kStageConvert],
                                                                            g->r);
        SA3K_LAUNCHED();
    }
    if (g->merged) {
        double bytes = 0.0;
        for (sa3k_lin* L : g->lins) bytes += (double)L->W->in * (double)L->W->out * (type_size(L->W->type) + 4.0);
        KernelScope ks(ctx, "group_merge", bytes);
        // one launch per element type present (blocks of other members exit at once)
        bool has[4] = {false, false, false, false};
        for (sa3k_lin* L : g->lins) has[L->W->type == SA3K_TYPE_F32 ? 0 : L->W->type == SA3K_TYPE_F16 ? 1 : L->W->type == SA3K_TYPE_BF16 ? 2 : 3] = true;
        void (*kern[4])(const PrepDesc*, const int*, int, float) = {
            group_merge_kernel<SA3K_TYPE_F32>, group_merge_kernel<SA3K_TYPE_F16>, group_merge_kernel<SA3K_TYPE_BF16>,
            group_merge_kernel<SA3K_TYPE_Q8_0>};
        for (int t = 0; t < 4; ++t) {
            if (!has[t]) continue;
            kern[t]<<<(unsigned)g->blocks[kStageMerge], kThreads, 0, ctx->stream>>>(g->dev, g->block_member[kStageMerge],
                                                                                 g->r, g->s);
            SA3K_LAUNCHED();
        }
        return;
    }
    if (!g->dora) return;
    {
        double flops = 0.0;
        for (sa3k_lin* L : g->lins) flops += 2.0 * g->r * (double)L->W->in * (double)L->W->out;
        KernelScope ks(ctx, "group_pt", flops);
        if (g->f32) {
            // one launch per stored element type present (blocks of other members exit at once)
            bool has32 = false, has16 = false;
            for (sa3k_lin* L : g->lins) (L->W->type == SA3K_TYPE_F32 ? has32 : has16) = true;
            if (has32) {
                group_pt_f32_kernel<SA3K_TYPE_F32><<<(unsigned)g->blocks[kStagePt], kThreads, 0, ctx->stream>>>(
                    g->dev, g->block_member[kStagePt], g->r);
                SA3K_LAUNCHED();
            }
            if (has16) {
                group_pt_f32_kernel<SA3K_TYPE_F16><<<(unsigned)g->blocks[kStagePt], kThreads, 0, ctx->stream>>>(
                    g->dev, g->block_member[kStagePt], g->r);
                SA3K_LAUNCHED();
            }
        } else {
            auto* kern = g->r > 16 ? group_pt_kernel<true> : group_pt_kernel<false>;
            kern<<<(unsigned)g->blocks[kStagePt], kThreads, 0, ctx->stream>>>(g->dev, g->block_member[kStagePt], g->r);
            SA3K_LAUNCHED();
        }
    }
    {
        KernelScope ks(ctx, "group_gram");
        double* part = reinterpret_cast<double*>(reduce_workspace(ctx, (size_t)g->blocks[kStageGram] * 1024 * sizeof(double)));
        group_gram_part_kernel<<<(unsigned)g->blocks[kStageGram], kThreads, 0, ctx->stream>>>(
            g->dev, g->block_member[kStageGram], g->r, part);
        SA3K_LAUNCHED();
        group_gram_sum_kernel<<<(unsigned)g->n, kThreads, 0, ctx->stream>>>(g->dev, g->r, part);
        SA3K_LAUNCHED();
    }
    {
        KernelScope ks(ctx, "group_dora_terms");
        group_dora_terms_kernel<<<(unsigned)g->blocks[kStageTerms], kThreads, 0, ctx->stream>>>(
            g->dev, g->block_member[kStageTerms], g->r, g->s);
        SA3K_LAUNCHED();
    }
}

// ---------------------------------------------------------------- stacked products
struct LinStack {
    std::vector<sa3k_lin*> lins;
    int64_t in = 0, out = 0, max_tokens = 0;
    int r = 0;
    void *Wm = nullptr, *Ac = nullptr, *U = nullptr, *H = nullptr, *Xb = nullptr;
    float *d = nullptr, *Y = nullptr;
};

void lin_stack_free(LinStack* s) {
    if (!s) return;
    for (void* p : {s->Wm, s->Ac, s->U, s->H, s->Xb, (void*)s->d, (void*)s->Y})
        if (p) (void)hipFree(p);
    delete s;
}

LinStack* lin_stack_create(sa3k_ctx* ctx, sa3k_lin* const* lins, int n) {
    SA3K_REQUIRE(n > 0 && lins, "empty stack");
    // eligible: merged refresh on, bf16 adapted linears of one shape, rank and token budget, not yet
    // prepared, stacked weights below 2 GiB (buffer descriptors); otherwise no stack (null)
    if (!ctx->lin_merge) return nullptr;
    const sa3k_lin* L0 = lins[0];
    for (int i = 0; i < n; ++i) {
        const sa3k_lin* L = lins[i];
        if (L->prec != SA3K_PREC_BF16 || L->rank != L0->rank || L0->rank <= 0 || L->W->in != L0->W->in ||
            L->W->out != L0->W->out || L->max_tokens != L0->max_tokens || L->ext != 0 || L->Wm || L->solo)
            return nullptr;
    }
    if (L0->W->out % 8 != 0 || (int64_t)n * L0->W->out * L0->W->in * 2 >= ((int64_t)1 << 31)) return nullptr;
    LinStack* st = new LinStack();
    try {
        st->in = L0->W->in;
        st->out = L0->W->out;
        st->r = L0->rank;
        st->max_tokens = L0->max_tokens;
        const int64_t cols = (int64_t)n * st->out, rcols = (int64_t)n * st->r;
        st->Wm = dev_alloc<bf16>(cols * st->in);
        st->Ac = dev_alloc<bf16>(rcols * st->in);
        st->d = dev_alloc<float>(cols);
        st->U = dev_alloc<bf16>(st->max_tokens * cols);
        st->H = dev_alloc<bf16>(st->max_tokens * rcols);
        st->Y = dev_alloc<float>(st->max_tokens * cols);
        st->Xb = dev_alloc<bf16>(st->max_tokens * st->in);
        for (int i = 0; i < n; ++i) {
            sa3k_lin* L = lins[i];
            for (void* p : {L->Ac, (void*)L->d, L->U, L->Hc})
                if (p) SA3K_HIP(hipFree(p));
            L->Ac = static_cast<bf16*>(st->Ac) + (int64_t)i * st->r * st->in;
            L->d = st->d + (int64_t)i * st->out;
            L->Wm = static_cast<bf16*>(st->Wm) + (int64_t)i * st->out * st->in;
            L->U = static_cast<bf16*>(st->U) + (int64_t)i * st->out;
            L->Hc = static_cast<bf16*>(st->H) + (int64_t)i * st->r;
            L->ldu = cols;
            L->ldh = rcols;
            L->ext = kExtAc | kExtD | kExtWm | kExtU | kExtHc;
            st->lins.push_back(L);
        }
    } catch (...) {
        lin_stack_free(st);
        throw;
    }
    return st;
}

const float* lin_stack_forward(sa3k_ctx* ctx, LinStack* st, const float* X, int64_t N) {
    const int n = (int)st->lins.size();
    const sa3k_lin* L0 = st->lins[0];
    SA3K_REQUIRE(N > 0 && N <= st->max_tokens, "tokens exceed the stack's budget");
    for (const sa3k_lin* L : st->lins)
        SA3K_REQUIRE(L->merged && L->dora == L0->dora && L->s == L0->s,
                     "stack members must be prepared merged, with one scale and adapter kind");
    const int64_t cols = (int64_t)n * st->out, rcols = (int64_t)n * st->r;
    {
        const int64_t e = N * st->in;
        KernelScope ks(ctx, "lin_stack_cvt_x");
        launch_k(ctx, true, cvt_kernel<bf16>, dim3((unsigned)ceil_div(e, kThreads)), dim3(kThreads), 0, X,
                 static_cast<bf16*>(st->Xb), e, 1.0f);
        SA3K_LAUNCHED();
    }
    // Y_i = d_i (.) (X W_eff,i^T) for every member as one product over the stacked W_eff, with
    // s X A_i^T of every member as the extra columns
    GemmDesc g;
    g.prec = SA3K_PREC_BF16; g.a_src = SRC_BF16; g.b_src = SRC_BF16;
    g.A = st->Xb; g.lda = st->in;
    g.B = st->Wm; g.ldb = st->in;
    g.Nx = rcols; g.Bx = st->Ac; g.ldbx = st->in; g.alpha_x = L0->s; g.Cbn = static_cast<bf16*>(st->H); g.ldcn = rcols;
    g.M = N; g.N = cols; g.K = st->in; g.alpha = 1.0f;
    g.colscale = L0->dora ? st->d : nullptr;
    g.C = st->Y; g.ldc = cols;
    g.ldu = cols;
    if (L0->dora) g.Ub = static_cast<bf16*>(st->U);
    gemm_run(ctx, g, "lin_stack_fwd");
    for (sa3k_lin* L : st->lins) L->saved_tokens = N;
    return st->Y;
}

int64_t lin_stack_ld(const LinStack* st) { return (int64_t)st->lins.size() * st->out; }
const float* lin_stack_y(const LinStack* st) { return st->Y; }

}  // namespace sa3k

// ------------------------------------------------------------------------------------ C ABI
extern "C" {

SA3K_API int sa3k_weight_create(sa3k_ctx* ctx, int type, int64_t in, int64_t out, const void* data,
                                int data_on_device, sa3k_weight** out_w) {
    return sa3k_guard(ctx, "sa3k_weight_create", [&] {
        SA3K_REQUIRE(out_w && data, "null pointer");
        *out_w = nullptr;
        SA3K_REQUIRE(in > 0 && out > 0, "weight extents must be positive");
        SA3K_REQUIRE(type == SA3K_TYPE_F32 || type == SA3K_TYPE_F16 || type == SA3K_TYPE_BF16 ||
                     type == SA3K_TYPE_Q8_0, "unsupported weight type");
        SA3K_REQUIRE(in % 64 == 0, "weight input dimension must be a multiple of 64");
        SA3K_REQUIRE(type != SA3K_TYPE_Q8_0 || out % 32 == 0, "Q8_0 output dimension must be a multiple of 32");
        SA3K_REQUIRE(out % 8 == 0, "weight output dimension must be a multiple of 8");
        sa3k_weight* w = new sa3k_weight();
        w->type = type; w->in = in; w->out = out;
        try {
            const int64_t n = in * out;
            const size_t raw_bytes = type == SA3K_TYPE_Q8_0 ? (size_t)(n / 32) * 34 : (size_t)n * type_size(type);
            const void* src = data;
            void* staging = nullptr;
            if (!data_on_device) {
                SA3K_HIP(hipMalloc(&staging, raw_bytes));
                SA3K_HIP(hipMemcpyAsync(staging, data, raw_bytes, hipMemcpyHostToDevice, ctx->stream));
                sa3k_note_main(ctx);
                src = staging;
            }
            if (type == SA3K_TYPE_Q8_0) {
                w->w = dev_alloc<int8_t>(n);
                w->ws = dev_alloc<uint16_t>(n / 32);
                w->wt = dev_alloc<int8_t>(n);
                w->wts = dev_alloc<uint16_t>(n / 32);
                q8_split_kernel<<<(unsigned)ceil_div(n / 32, kThreads), kThreads, 0, ctx->stream>>>(
                    static_cast<const uint16_t*>(src), static_cast<int8_t*>(w->w), static_cast<uint16_t*>(w->ws), n / 32);
                SA3K_LAUNCHED();
                transpose<int8_t>(ctx, static_cast<int8_t*>(w->w), static_cast<int8_t*>(w->wt), out, in);
                transpose<uint16_t>(ctx, static_cast<uint16_t*>(w->ws), static_cast<uint16_t*>(w->wts), out, in / 32);
            } else {
                const size_t es = type_size(type);
                SA3K_HIP(hipMalloc(&w->w, (size_t)n * es));
                SA3K_HIP(hipMalloc(&w->wt, (size_t)n * es));
                SA3K_HIP(hipMemcpyAsync(w->w, src, (size_t)n * es, hipMemcpyDeviceToDevice, ctx->stream));
                sa3k_note_main(ctx);
                if (es == 4) transpose<uint32_t>(ctx, static_cast<uint32_t*>(w->w), static_cast<uint32_t*>(w->wt), out, in);
                else transpose<uint16_t>(ctx, static_cast<uint16_t*>(w->w), static_cast<uint16_t*>(w->wt), out, in);
            }
            if (type != SA3K_TYPE_BF16) {
                w->wb = dev_alloc<bf16>(n);
                w->wbt = dev_alloc<bf16>(n);
                decode_bf16_kernel<<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(*w, static_cast<bf16*>(w->wb));
                SA3K_LAUNCHED();
                transpose<uint16_t>(ctx, static_cast<uint16_t*>(w->wb), static_cast<uint16_t*>(w->wbt), out, in);
            }
            SA3K_HIP(hipStreamSynchronize(ctx->stream));
            if (staging) SA3K_HIP(hipFree(staging));
        } catch (...) {
            free_weight(w);
            throw;
        }
        *out_w = w;
    });
}

SA3K_API int sa3k_weight_drop_working_copy(sa3k_ctx* ctx, sa3k_weight* w) {
    return sa3k_guard(ctx, "sa3k_weight_drop_working_copy", [&] {
        SA3K_REQUIRE(w != nullptr, "null weight");
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        if (w->wb) SA3K_HIP(hipFree(w->wb));
        if (w->wbt) SA3K_HIP(hipFree(w->wbt));
        w->wb = w->wbt = nullptr;
    });
}

SA3K_API int sa3k_weight_destroy(sa3k_ctx* ctx, sa3k_weight* w) {
    return sa3k_guard(ctx, "sa3k_weight_destroy", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        free_weight(w);
    });
}

SA3K_API int sa3k_weight_row_norm_sq(sa3k_ctx* ctx, const sa3k_weight* w, float eps, float* nsq) {
    return sa3k_guard(ctx, "sa3k_weight_row_norm_sq", [&] {
        SA3K_REQUIRE(w && nsq, "null pointer");
        KernelScope ks(ctx, "weight_row_norm");
        row_norm_kernel<<<(unsigned)w->out, kThreads, 0, ctx->stream>>>(*w, eps, 0, nsq);
        SA3K_LAUNCHED();
    });
}

SA3K_API int sa3k_row_norms(sa3k_ctx* ctx, int type, int64_t in, int64_t out, const void* W, int mode, float eps,
                            float* result) {
    return sa3k_guard(ctx, "sa3k_row_norms", [&] {
        SA3K_REQUIRE(W && result && in > 0 && out > 0 && (mode == 0 || mode == 1), "bad arguments");
        SA3K_REQUIRE(type == SA3K_TYPE_F32 || type == SA3K_TYPE_F16 || type == SA3K_TYPE_BF16,
                     "row norms of an element type (f32 / f16 / bf16)");
        sa3k_weight w;   // a view: no copy, no working copies
        w.type = type; w.in = in; w.out = out; w.w = const_cast<void*>(W);
        KernelScope ks(ctx, "weight_row_norm");
        row_norm_kernel<<<(unsigned)out, kThreads, 0, ctx->stream>>>(w, eps, mode == 0 ? 1 : 0, result);
        SA3K_LAUNCHED();
    });
}

SA3K_API int sa3k_weight_row_norms(sa3k_ctx* ctx, const sa3k_weight* w, float* norms) {
    return sa3k_guard(ctx, "sa3k_weight_row_norms", [&] {
        SA3K_REQUIRE(w && norms, "null pointer");
        KernelScope ks(ctx, "weight_row_norm");
        row_norm_kernel<<<(unsigned)w->out, kThreads, 0, ctx->stream>>>(*w, 0.0f, 1, norms);
        SA3K_LAUNCHED();
    });
}

SA3K_API int sa3k_lin_create(sa3k_ctx* ctx, const sa3k_weight* W, int rank, int prec, int64_t max_tokens,
                             sa3k_lin** out_l) {
    return sa3k_guard(ctx, "sa3k_lin_create", [&] {
        SA3K_REQUIRE(W && out_l, "null pointer");
        *out_l = nullptr;
        SA3K_REQUIRE(rank >= 0 && rank <= 32 && rank % 8 == 0, "rank must be 0, 8, 16, 24 or 32");
        SA3K_REQUIRE(prec == SA3K_PREC_BF16 || prec == SA3K_PREC_F32, "unknown precision");
        SA3K_REQUIRE(prec == SA3K_PREC_BF16 || W->type == SA3K_TYPE_F32 || W->type == SA3K_TYPE_F16,
                     "f32 precision needs an f32 or f16 weight");
        SA3K_REQUIRE(prec == SA3K_PREC_BF16 || rank % 4 == 0, "rank");
        SA3K_REQUIRE(max_tokens > 0, "max_tokens must be positive");
        sa3k_lin* L = new sa3k_lin();
        L->W = W; L->rank = rank; L->prec = prec; L->max_tokens = max_tokens;
        L->ct = prec == SA3K_PREC_BF16 ? 2 : 4;
        try {
            const int64_t in = W->in, out = W->out, r = std::max(rank, 1);
            auto ct_alloc = [&](int64_t n) { void* p = nullptr; SA3K_HIP(hipMalloc(&p, (size_t)std::max<int64_t>(n, 1) * L->ct)); return p; };
            L->Ac = ct_alloc(r * in); L->At = ct_alloc(r * in);
            L->Bc = ct_alloc(r * out); L->Bt = ct_alloc(r * out);
            L->Pt = dev_alloc<float>(r * out); L->G = dev_alloc<float>(r * r); L->BG = dev_alloc<float>(r * out);
            L->nsq = dev_alloc<float>(out); L->d = dev_alloc<float>(out);
            L->Hc = ct_alloc(max_tokens * r); L->U = ct_alloc(max_tokens * out);
            L->dU = ct_alloc(max_tokens * out); L->sdUB = ct_alloc(max_tokens * r);
            if (prec == SA3K_PREC_BF16) L->Xb = dev_alloc<bf16>(max_tokens * in);
            L->gd = dev_alloc<float>(out); L->gn = dev_alloc<float>(out);
            L->Ax = ct_alloc(r * out); L->A2x = ct_alloc(r * r);
            L->red = dev_alloc<float>(33 * out);
        } catch (...) {
            free_lin(L);
            throw;
        }
        *out_l = L;
    });
}

SA3K_API int sa3k_lin_destroy(sa3k_ctx* ctx, sa3k_lin* L) {
    return sa3k_guard(ctx, "sa3k_lin_destroy", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        free_lin(L);
    });
}

SA3K_API int sa3k_lin_prepare(sa3k_ctx* ctx, sa3k_lin* L, const float* A, const float* B, float scale, int dora,
                              const float* magnitude, const float* base_norm_sq) {
    return sa3k_guard(ctx, "sa3k_lin_prepare", [&] {
        SA3K_REQUIRE(L != nullptr, "null linear");
        const int64_t in = L->W->in, out = L->W->out;
        const int r = L->rank;
        L->s = scale;
        L->dora = dora ? 1 : 0;
        L->B = B;
        L->mag = magnitude;
        if (r == 0) {
            SA3K_REQUIRE(!dora, "dora needs a rank > 0 adapter");
            return;
        }
        SA3K_REQUIRE(A && B, "adapter A/B are null");
        SA3K_REQUIRE(!dora || (magnitude && base_norm_sq), "dora needs magnitude and base_norm_sq");
        const bool bf = L->prec == SA3K_PREC_BF16;
        L->merged = 0;
        if (bf && ctx->lin_merge && out % 16 == 0) {
            // the merged refresh through a one-member group, rebuilt when the adapter changes
            const float* key[4] = {A, B, dora ? magnitude : nullptr, dora ? base_norm_sq : nullptr};
            if (!L->solo || !std::equal(key, key + 4, L->solo_key) || L->solo_s != scale || L->solo_dora != dora) {
                if (L->solo) {
                    SA3K_HIP(hipStreamSynchronize(ctx->stream));
                    lin_group_free(L->solo);
                    L->solo = nullptr;
                }
                sa3k_lin* one = L;
                L->solo = lin_group_create(ctx, &one, 1, &key[0], &key[1], &key[2], &key[3], scale, dora);
                std::copy(key, key + 4, L->solo_key);
                L->solo_s = scale;
                L->solo_dora = dora;
            }
            lin_group_prepare(ctx, L->solo);
            return;
        }
        KernelScope ks(ctx, "lin_prepare");
        auto cvt = [&](const float* src, void* dst, int64_t n) {
            if (bf) cvt_kernel<bf16><<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(src, static_cast<bf16*>(dst), n, 1.0f);
            else cvt_kernel<float><<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(src, static_cast<float*>(dst), n, 1.0f);
            SA3K_LAUNCHED();
        };
        auto cvt_t = [&](const float* src, void* dst, int64_t rows, int64_t cols) {
            const int64_t n = rows * cols;
            if (bf) cvt_t_kernel<bf16><<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(src, static_cast<bf16*>(dst), rows, cols);
            else cvt_t_kernel<float><<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(src, static_cast<float*>(dst), rows, cols);
            SA3K_LAUNCHED();
        };
        cvt(A, L->Ac, (int64_t)r * in);
        cvt_t(A, L->At, r, in);
        cvt(B, L->Bc, (int64_t)out * r);
        cvt_t(B, L->Bt, out, r);
        if (!dora) return;
        // P^T = A W^T  [r][out]: streams W once through the forward weight loader
        const WOp wo = weight_operand(L->W, bf, false);
        GemmDesc g;
        g.prec = L->prec; g.a_src = bf ? SRC_BF16 : SRC_F32; g.b_src = wo.src;
        g.A = L->Ac; g.lda = in; g.B = wo.p; g.ldb = wo.ld; g.Bs = wo.s; g.ldbs = wo.lds;
        g.M = r; g.N = out; g.K = in; g.C = L->Pt; g.ldc = out;
        gemm_run(ctx, g, "lin_prepare_p");
        gram_kernel<<<(unsigned)(r * r), kThreads, 0, ctx->stream>>>(A, in, r, L->G);
        SA3K_LAUNCHED();
        dora_terms_kernel<<<(unsigned)ceil_div(out, 8), kThreads, 0, ctx->stream>>>(
            L->Pt, B, L->G, base_norm_sq, magnitude, out, r, scale, L->BG, L->nsq, L->d);
        SA3K_LAUNCHED();
    });
}

SA3K_API int sa3k_lin_forward(sa3k_ctx* ctx, sa3k_lin* L, int x_type, const void* X, int64_t N, const float* bias,
                              float* Y) {
    return sa3k_guard(ctx, "sa3k_lin_forward", [&] {
        SA3K_REQUIRE(L && X && Y, "null pointer");
        SA3K_REQUIRE(N > 0 && N <= L->max_tokens, "token count exceeds the linear's max_tokens");
        SA3K_REQUIRE(x_type == SA3K_TYPE_F32 || (x_type == SA3K_TYPE_BF16 && L->prec == SA3K_PREC_BF16),
                     "activation type must be f32 (or bf16 with bf16 precision)");
        const int xs = x_type == SA3K_TYPE_F32 ? SRC_F32 : SRC_BF16;
        if (L->prec == SA3K_PREC_BF16) lin_forward_t<bf16>(ctx, L, xs, X, N, bias, Y);
        else lin_forward_t<float>(ctx, L, xs, X, N, bias, Y);
    });
}

}  // extern "C"

// sa3k_lin_forward of the FFN up-projection (bf16 activations) that also writes g = bf16(val *
// silu(glu)) of Y = [val | glu] from its GEMM epilogue when bit 0 of the option epi_fuse is set and
// the chosen kernel allows it; returns whether it did (else the caller applies SwiGLU to Y itself)
bool sa3k::lin_forward_swiglu(sa3k_ctx* ctx, sa3k_lin* L, const bf16* X, int64_t N, const float* bias, float* Y,
                              bf16* Yb, bf16* g) {
    SA3K_REQUIRE(L && X && Y && g, "null pointer");
    SA3K_REQUIRE(N > 0 && N <= L->max_tokens, "token count exceeds the linear's max_tokens");
    SA3K_REQUIRE(L->prec == SA3K_PREC_BF16 && L->ext == 0, "the fused SwiGLU needs a bf16 linear outside a stack");
    int done = 0;
    LinEpi e;
    e.sw_g = (ctx->epi_fuse & 1) ? g : nullptr;
    e.Yb = Yb;
    e.done = &done;
    lin_forward_t<bf16>(ctx, L, SRC_BF16, X, N, bias, Y, &e);
    return done != 0;
}

// sa3k_lin_forward of an attention projection (bf16 activations) that also prepares the heads
// (HeadPrep) from its GEMM epilogue when bit 1 of the option epi_fuse is set and the chosen kernel
// allows it; returns whether it did (else the caller prepares them from Y)
bool sa3k::lin_forward_headprep(sa3k_ctx* ctx, sa3k_lin* L, const bf16* X, int64_t N, float* Y, bf16* Yb,
                                const HeadPrep& hp) {
    SA3K_REQUIRE(L && X && Y, "null pointer");
    SA3K_REQUIRE(N > 0 && N <= L->max_tokens, "token count exceeds the linear's max_tokens");
    SA3K_REQUIRE(L->prec == SA3K_PREC_BF16 && L->ext == 0, "the head preparation needs a bf16 linear outside a stack");
    int done = 0;
    LinEpi e;
    e.hp = (ctx->epi_fuse & 2) ? &hp : nullptr;
    e.Yb = Yb;
    e.done = &done;
    lin_forward_t<bf16>(ctx, L, SRC_BF16, X, N, nullptr, Y, &e);
    return done != 0;
}

extern "C" {

SA3K_API int sa3k_lin_backward(sa3k_ctx* ctx, sa3k_lin* L, int x_type, const void* X, int64_t N, const float* dY,
                               float* dX, int dx_accumulate, float* dA, float* dB, float* dm) {
    return sa3k_guard(ctx, "sa3k_lin_backward", [&] {
        SA3K_REQUIRE(L && X && dY, "null pointer");
        SA3K_REQUIRE(N == L->saved_tokens, "backward must follow a forward over the same tokens");
        SA3K_REQUIRE(L->rank == 0 || (dA && dB), "adapter gradients need dA/dB buffers");
        SA3K_REQUIRE(!L->dora || dm, "dora needs a magnitude gradient buffer");
        SA3K_REQUIRE(x_type == SA3K_TYPE_F32 || (x_type == SA3K_TYPE_BF16 && L->prec == SA3K_PREC_BF16),
                     "activation type must be f32 (or bf16 with bf16 precision)");
        const int xs = x_type == SA3K_TYPE_F32 ? SRC_F32 : SRC_BF16;
        const int r = L->rank;
        if (L->prec == SA3K_PREC_BF16) {
            if (r <= 16) lin_backward_t<bf16, 16>(ctx, L, xs, X, N, dY, dX, dx_accumulate, dA, dB, dm);
            else lin_backward_t<bf16, 32>(ctx, L, xs, X, N, dY, dX, dx_accumulate, dA, dB, dm);
        } else {
            if (r <= 16) lin_backward_t<float, 16>(ctx, L, xs, X, N, dY, dX, dx_accumulate, dA, dB, dm);
            else lin_backward_t<float, 32>(ctx, L, xs, X, N, dY, dX, dx_accumulate, dA, dB, dm);
        }
    });
}

}  // extern "C"
