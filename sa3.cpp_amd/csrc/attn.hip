// K5: differential attention, flash-style, on bf16 MFMA (head_dim 64).
//
// Reference: dit_diff_attn (src/dit.h:151-158) over nn::sdpa (src/nn.h:135-144): per (batch,
// head) O = softmax(Q1 K1^T s) V - softmax(Q2 K2^T s) V, materialised [S x S] scores in ggml.
// Here nothing of size S x S ever leaves the CU:
//   forward   one pass over key blocks keeps both branches' online-softmax state and shares the
//             V tile; writes O (token-major bf16, the out-projection's input), the normalised
//             branch outputs O1, O2 and the per-query log2-sum-exp of each branch;
//   backward  Dn_i = rowsum(dO * O_i) first (also re-lays dO head-major in bf16), then two
//             recompute kernels: one per key block (dK1, dK2, dV; loops over queries) and one
//             per query block (dQ1, dQ2; loops over keys) -- no atomics, deterministic.
// With dO_2 = -dO: dS_1 = P1 (dP - Dn1), dS_2 = -P2 (dP - Dn2), dP = dO V^T, dV = (P1 - P2)^T dO.
//
// MFMA layout (v_mfma_f32_16x16x32_bf16): scores are computed transposed, S^T = K Q^T, so that a
// lane holds one query (lane % 16) and 4 keys per 16-key tile; two adjacent key tiles give the 8
// key-values that lane feeds as the A operand of P V. The operand on the other side (V for P V,
// Q and dO for dK and dV, K for dQ) contracts over the tile's row index; it is read with
// ds_read_b64_tr_b16 straight from the row-major tile in the same key order, so both operands
// agree on K order. The dK/dV kernel computes S = Q K^T instead (lane = one key).
//
// Tiles are [64 rows][64] bf16, 128-byte XOR-swizzled LDS rows, filled by buffer_load ... lds DMA
// through a per-tile buffer descriptor whose extent ends at the last valid row, so rows past the
// sequence read as zeros. Two LDS stages: the DMA of block i+1 runs while block i is computed.
//
// window > 0 keeps keys with |q - k| <= window/2 (self-attention only); 0 is dense.
#include "headprep.h"
#include "sa3k_internal.h"

#include <algorithm>
#include <type_traits>

namespace sa3k {
float* gemm_workspace_bytes(sa3k_ctx* ctx, size_t bytes);   // gemm.hip: context-owned scratch
}

namespace {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr int kThreads = 256;
constexpr int HD = 64;          // head dim
constexpr int BLK = 64;         // queries / keys per block
constexpr int ROW = 128;        // bytes per [row][64] bf16 LDS row (swizzled, unpadded)
constexpr float kLog2e = 1.4426950408889634f;

// XOR swizzle of the eight 16-byte chunks of a 128-byte LDS row: rows r and r^1 sit in different
// bank halves, and the chunk XOR is a linear map of a = (r>>1)&7, s = (a2, a1^a2, a0) as bits
// (s0, s1, s2). Every read pattern of these kernels is bank-conflict-free with it on gfx950: the
// ds_read_b128 row reads (lane l: chunk c + l/16 of row l%16, or chunk c + l/32 of row l%32) and the
// ds_read_b64_tr_b16 reads of four or eight consecutive rows per 16 lanes (ld_tr below). Measured
// with SQ_LDS_BANK_CONFLICT over every invertible map of a: 32 of the 168 serve all four patterns
// in one pass per lane group; the bit permutation (a0, a2, a1) used before cost 2 extra cycles per
// transposed read, (r&7)^(r>>3&1) before it 3.2 per row read. (The kernels are latency-bound: the
// conflict-free map made the forwards 1-2% faster and left the backward within noise.)
__device__ __forceinline__ int swz(int r) {
    const int a = (r >> 1) & 7;
    return ((a >> 2) & 1) | ((((a >> 1) ^ (a >> 2)) & 1) << 1) | ((a & 1) << 2);
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16-byte chunk c (8 dims) of row r in a swizzled [64][64] tile
__device__ __forceinline__ bf16x8 ld_row(const char* t, int r, int c) {
    return *reinterpret_cast<const bf16x8*>(t + r * ROW + ((c ^ swz(r)) << 4));
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Transposed read (ds_read_b64_tr_b16) of a swizzled tile: every 16-lane group returns, in lane
// j of the group, the 4 values T[k0 .. k0+3][n0 + j]. Lane j of the group addresses row k0 + j/4,
// columns n0 + 4*(j%4) .. +3 (the instruction hands element i%4 of the chunks of lanes
// i/4, i/4+4, i/4+8, i/4+12 to lane i). k0 and n0 may differ between the four groups.
__device__ __forceinline__ bf16x4 ld_tr(const char* t, int k0, int n0, int lane) {
    const int j = lane & 15, row = k0 + (j >> 2), n = n0 + 4 * (j & 3);
    const char* a = t + row * ROW + (((n >> 3) ^ swz(row)) << 4) + (n & 7) * 2;
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(
        (lds_ptr_t)a)));
}
__device__ __forceinline__ bf16x8 cat44(bf16x4 a, bf16x4 b) {
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Raw buffer descriptor over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const unsigned long long a = (unsigned long long)(uintptr_t)base;
    u32x4 r;
    // the descriptor lives in SGPRs: make its (wave-uniform) words provably uniform
    r.x = __builtin_amdgcn_readfirstlane((unsigned)a);
    r.y = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32) & 0xffffu);   // stride 0
    r.z = __builtin_amdgcn_readfirstlane(bytes);                           // num_records
    r.w = 0x00020000u;                                                     // 32-bit format, no swizzle
    return r;
}

// Issue the DMA of rows row0 .. row0+63 of a [nrows][64] bf16 matrix into a swizzled LDS tile
// (512 16-byte slots, two per thread; slot s holds row s/8, logical chunk (s%8) ^ swz(row)).
// Inline asm so that the compiler's waits do not drain the DMA before unrelated LDS reads; the
// kernels order it with vmcnt waits and barriers.
__device__ __forceinline__ void tile_dma(const bf16* base, int nrows, int row0, const char* lds_tile, int tid,
                                         int wave) {
    const int valid = max(0, min(BLK, nrows - row0));
    const u32x4 rs = buffer_rsrc(base + (int64_t)row0 * HD, (uint32_t)valid * ROW);
    const uint32_t tile = (uint32_t)(uintptr_t)(lds_ptr_t)lds_tile;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int sl = q * kThreads + tid, row = sl >> 3, kc = (sl & 7) ^ swz(row);
        const uint32_t voff = (uint32_t)(row * ROW + kc * 16);
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(tile + (uint32_t)((q * kThreads + wave * 64) * 16));
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(rs)
                     : "memory");
    }
}
// DMA of 64 floats v[i0 .. i0+63] (zeros past n) into LDS, by one wave (one dword per lane)
__device__ __forceinline__ void vec_dma(const float* v, int n, int i0, const float* lds_vec, int lane) {
    const int valid = max(0, min(BLK, n - i0));
    const u32x4 rs = buffer_rsrc(v + i0, (uint32_t)valid * 4);
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds_vec);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0), "v"((uint32_t)lane * 4),
                 "s"(rs)
                 : "memory");
}
// this wave's DMAs have landed; then a barrier makes every wave's visible
__device__ __forceinline__ void dma_wait_all() {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// 2^x on the hardware's exp unit (v_exp_f32, no denormal rescaling: results below 2^-126, the
// weights of keys more than ~87 nats under the row maximum, flush to zero)
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// The keys one query sees form the range [lo, lo + n): |q - k| <= window/2 (window > 0) and
// k < nk. With it a visibility test is one unsigned compare: (unsigned)(k - lo) < n.
struct Span {
    int lo, n;
};
__device__ __forceinline__ Span visible(int q, int nk, int window) {
    if (window <= 0) return Span{0, nk};
    const int half = window / 2, lo = max(0, q - half), hi = min(nk - 1, q + half);
    return Span{lo, max(0, hi - lo + 1)};
}
// every (q, k) of query block qb x key block kb is visible and in range (a block-uniform test)
__device__ __forceinline__ bool block_full(int qb, int kb, int nq, int nk, int window) {
    if ((qb + 1) * BLK > nq || (kb + 1) * BLK > nk) return false;
    if (window <= 0) return true;
    const int far = max(qb * BLK + BLK - 1 - kb * BLK, kb * BLK + BLK - 1 - qb * BLK);
    return 2 * far <= window;
}

// key/query block range [lo, hi) that can interact with block b under the window
__device__ __forceinline__ void band_range(int b, int n_other, int window, int& lo, int& hi) {
    const int nb = (n_other + BLK - 1) / BLK;
    lo = 0;
    hi = nb;
    if (window > 0) {
        const int half = window / 2;
        lo = max(0, (b * BLK - half) / BLK);
        hi = min(nb, (b * BLK + BLK - 1 + half) / BLK + 1);
    }
}

// This workgroup's (block, bh) from its place in dispatch order (x fastest, then y): the blocks
// go out from the middle of the sequence to its ends, every (batch, head) of one block before the
// next block. Under a window the middle blocks meet the most key (query) blocks and the end ones
// the fewest, so the grid starts with the longest workgroups and ends with the shortest, and the
// last wave of workgroups is short. Consecutive workgroups differ in bh, so with BH a multiple of 8
// every workgroup of one (batch, head) runs on the same XCD (dispatch deals them out round-robin)
// and shares its L2.
__device__ __forceinline__ void heavy_first(int& blk, int& bh) {
    const int n = gridDim.x, BH = gridDim.y;
    const int L = blockIdx.x + n * blockIdx.y;
    const int k = L / BH;
    bh = L - k * BH;
    blk = (k & 1) ? n / 2 - (k + 1) / 2 : n / 2 + k / 2;
}

// ------------------------------------------------------------------------------------ forward
struct FwdArgs {
    const bf16 *q1, *k1, *q2, *k2, *v;   // [BH][S][64]
    int H, Sq, Sk, window;
    float scale;
    bf16* o;             // [B][Sq][H*64] token-major
    bf16 *o1, *o2;       // [BH][Sq][64] normalised branch outputs
    float *lse1, *lse2;  // [BH][Sq] log2-sum-exp of scale*log2e*scores
};

__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(FwdArgs a) {
    __shared__ __attribute__((aligned(1024))) char lds[2 * 3 * BLK * ROW];   // 2 stages x {K1, K2, V}
    int qb, bh;
    heavy_first(qb, bh);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, r = lane & 15;
    const int64_t qoff = (int64_t)bh * a.Sq * HD, koff = (int64_t)bh * a.Sk * HD;
    const int qrow = qb * BLK + w * 16 + r;        // this lane's query for the S^T layout
    const float c = a.scale * kLog2e;
    const Span sp = visible(qrow, a.Sk, a.window);

    bf16x8 q1f[2], q2f[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        uint4 z = make_uint4(0, 0, 0, 0), u1 = z, u2 = z;
        if (qrow < a.Sq) {
            u1 = *reinterpret_cast<const uint4*>(a.q1 + qoff + (int64_t)qrow * HD + ks * 32 + g * 8);
            u2 = *reinterpret_cast<const uint4*>(a.q2 + qoff + (int64_t)qrow * HD + ks * 32 + g * 8);
        }
        q1f[ks] = __builtin_bit_cast(bf16x8, u1);
        q2f[ks] = __builtin_bit_cast(bf16x8, u2);
    }
    f32x4 o1[4], o2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o1[i] = o2[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m1 = -INFINITY, m2 = -INFINITY, l1 = 0.f, l2 = 0.f;   // per lane: query qrow (l partial)

    int kb_lo, kb_hi;
    band_range(qb, a.Sk, a.window, kb_lo, kb_hi);
    auto issue = [&](int st, int kb) {
        char* t = lds + st * 3 * BLK * ROW;
        tile_dma(a.k1 + koff, a.Sk, kb * BLK, t, threadIdx.x, wave);
        tile_dma(a.k2 + koff, a.Sk, kb * BLK, t + BLK * ROW, threadIdx.x, wave);
        tile_dma(a.v + koff, a.Sk, kb * BLK, t + 2 * BLK * ROW, threadIdx.x, wave);
    };
    if (kb_lo < kb_hi) issue(0, kb_lo);
    for (int kb = kb_lo; kb < kb_hi; ++kb) {
        // no contraction of the score scaling into the exponent's subtraction: the row maximum's
        // weight must come out exactly 2^0 = 1
#pragma clang fp contract(off)
        const int st = (kb - kb_lo) & 1;
        dma_wait_all();   // block kb landed; every wave is done with block kb-1 (the other stage)
        if (kb + 1 < kb_hi) issue(st ^ 1, kb + 1);
        const char* k1s = lds + st * 3 * BLK * ROW;
        const char* k2s = k1s + BLK * ROW;
        const char* vs = k1s + 2 * BLK * ROW;
        // S^T tiles: keys kt*16 + 4g + v, query qrow
        f32x4 s1[4], s2[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            s1[kt] = s2[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                s1[kt] = mfma(ld_row(k1s, kt * 16 + r, ks * 4 + g), q1f[ks], s1[kt]);
                s2[kt] = mfma(ld_row(k2s, kt * 16 + r, ks * 4 + g), q2f[ks], s2[kt]);
            }
        }
        // The MFMA output layout is rows = 4*(lane/16)+v of the A operand (keys), col = lane%16
        // (queries); the A rows fed above were keys kt*16 + r, so output row index 4g+v is key
        // kt*16 + 4g + v and the column is query w*16 + r. Only blocks that cross the window's
        // edge or the sequence end are masked (a block-uniform branch).
        if (!block_full(qb, kb, a.Sq, a.Sk, a.window)) {
            const int rel = kb * BLK + 4 * g - sp.lo;   // key kt*16 + 4g + v, less lo, is rel + 16 kt + v
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const bool ok = (unsigned)(rel + 16 * kt + v) < (unsigned)sp.n;
                    s1[kt][v] = ok ? s1[kt][v] : -INFINITY;
                    s2[kt][v] = ok ? s2[kt][v] : -INFINITY;
                }
        }
        // scaled scores (rounded once, so the row maximum's weight is exactly 2^0 = 1) and maxima
        float mx1 = -INFINITY, mx2 = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                s1[kt][v] *= c;
                s2[kt][v] *= c;
                mx1 = fmaxf(mx1, s1[kt][v]);
                mx2 = fmaxf(mx2, s2[kt][v]);
            }
        mx1 = fmaxf(mx1, __shfl_xor(mx1, 16, 64));
        mx1 = fmaxf(mx1, __shfl_xor(mx1, 32, 64));
        mx2 = fmaxf(mx2, __shfl_xor(mx2, 16, 64));
        mx2 = fmaxf(mx2, __shfl_xor(mx2, 32, 64));
        const float mn1 = fmaxf(m1, mx1), mn2 = fmaxf(m2, mx2);
        const float base1 = mn1 == -INFINITY ? 0.f : mn1, base2 = mn2 == -INFINITY ? 0.f : mn2;
        const float al1 = ex2(m1 - base1), al2 = ex2(m2 - base2);   // 0 when m was -inf
        m1 = mn1;
        m2 = mn2;
        float ps1 = 0.f, ps2 = 0.f;
        bf16x8 p1[2], p2[2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float e1 = ex2(s1[kt][v] - base1), e2 = ex2(s2[kt][v] - base2);
                ps1 += e1;
                ps2 += e2;
                p1[kt >> 1][(kt & 1) * 4 + v] = (bf16)e1;
                p2[kt >> 1][(kt & 1) * 4 + v] = (bf16)e2;
            }
        l1 = l1 * al1 + ps1;
        l2 = l2 * al2 + ps2;
        // rescale O rows (queries w*16 + 4g + v) by their alpha (held by lane 4g+v)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float a1 = __shfl(al1, 4 * g + v, 64), a2 = __shfl(al2, 4 * g + v, 64);
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                o1[dt][v] *= a1;
                o2[dt][v] *= a2;
            }
        }
        // O += P V over two 32-key chunks: key(e) = 32c + (e < 4 ? 4g + e : 16 + 4g + e - 4)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const bf16x8 vb = cat44(ld_tr(vs, 32 * ch + 4 * g, dt * 16, lane), ld_tr(vs, 32 * ch + 16 + 4 * g, dt * 16, lane));
                o1[dt] = mfma(p1[ch], vb, o1[dt]);
                o2[dt] = mfma(p2[ch], vb, o2[dt]);
            }
    }
    // l: sum the four lane groups' partials (per query qrow)
    l1 += __shfl_xor(l1, 16, 64);
    l1 += __shfl_xor(l1, 32, 64);
    l2 += __shfl_xor(l2, 16, 64);
    l2 += __shfl_xor(l2, 32, 64);
    if (g == 0 && qrow < a.Sq) {
        a.lse1[(int64_t)bh * a.Sq + qrow] = m1 + log2f(l1);
        a.lse2[(int64_t)bh * a.Sq + qrow] = m2 + log2f(l2);
    }
    const int b = bh / a.H, h = bh % a.H;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float i1 = 1.0f / __shfl(l1, 4 * g + v, 64), i2 = 1.0f / __shfl(l2, 4 * g + v, 64);
        const int q = qb * BLK + w * 16 + 4 * g + v;
        if (q >= a.Sq) continue;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = dt * 16 + r;
            const float x1 = o1[dt][v] * i1, x2 = o2[dt][v] * i2;
            a.o1[qoff + (int64_t)q * HD + d] = (bf16)x1;
            a.o2[qoff + (int64_t)q * HD + d] = (bf16)x2;
            a.o[((int64_t)b * a.Sq + q) * (a.H * HD) + h * HD + d] = (bf16)(x1 - x2);
        }
    }
}

// Forward with one branch per wave, on 32x32x16 MFMA blocks: a workgroup takes 64 queries; waves 0
// and 1 compute branch 1 for queries 0..31 and 32..63, waves 2 and 3 branch 2 for the same queries,
// all from the same {K1, K2, V} tiles in LDS. Half the registers of a wave that carries both
// branches, so three waves share each SIMD and hide each other's MFMA, LDS and exp latency.
// Every product is computed transposed so that a lane owns one query throughout:
//   S^T[k][q] = K Q^T (A = K rows from LDS, B = Q in registers) -> lane l holds query l % 32 and
//               keys r(v) = 8 (v/4) + 4 (l/32) + v%4 of each 32-key half, v = 0..15;
//   O^T[d][q] += V^T P^T (A = V columns read transposed from LDS, B = P^T) -> lane l holds its own
//               query and dims 32 db + r(v), so the softmax rescale needs no lane exchange.
// P^T's K order is the order the lane already holds: K step j of a half takes values v = 8j..8j+7,
// i.e. keys 16j + 4 (l/32) + {0..3} and 16j + 8 + 4 (l/32) + {0..3}, and V^T is read in that order.
// The running maximum m moves only when a block's maximum exceeds it by more than kLazy (log2
// units), so the O rescale runs a few times per row instead of every block; the weights 2^(c s - m)
// stay below 2^kLazy, and O / l and lse = m + log2 l are the same quantities as with the exact
// maximum.
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
constexpr int QW = 32;          // queries per wave
constexpr float kLazy = 8.f;    // weights stay below 2^8
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(kThreads) void attn_fwd32_kernel(FwdArgs a) {
    __shared__ __attribute__((aligned(1024))) char lds[2 * 3 * BLK * ROW];   // 2 stages x {K1, K2, V}
    int qb, bh;
    heavy_first(qb, bh);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int br = wave >> 1;                // branch of this wave
    const int lane = threadIdx.x & 63, hl = lane >> 5, c32 = lane & 31;
    const int64_t qoff = (int64_t)bh * a.Sq * HD, koff = (int64_t)bh * a.Sk * HD;
    const int q0w = qb * BLK + (wave & 1) * QW;   // this wave's first query
    const int q = q0w + c32;                      // this lane's query
    const float c = a.scale * kLog2e;             // > 0 (checked by the host)
    const Span sp = visible(q, a.Sk, a.window);

    // Q as the B operand: query q, dims 16 ks + 8 (l/32) .. +7
    const bf16* qsrc = br ? a.q2 : a.q1;
    bf16x8 qf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        uint4 u = make_uint4(0, 0, 0, 0);
        if (q < a.Sq) u = *reinterpret_cast<const uint4*>(qsrc + qoff + (int64_t)q * HD + ks * 16 + hl * 8);
        qf[ks] = __builtin_bit_cast(bf16x8, u);
    }
    f32x16 o[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[i][v] = 0.f;
    float m = -INFINITY, l = 0.f;   // scaled running maximum of query q; this lane's partial sum

    // key blocks of the workgroup's 64 queries, and the keys this wave's 32 queries see
    int kb_lo, kb_hi;
    band_range(qb, a.Sk, a.window, kb_lo, kb_hi);
    int wlo = 0, whi = a.Sk;
    if (a.window > 0) {
        const int half = a.window / 2;
        wlo = max(0, q0w - half);
        whi = min(a.Sk, q0w + QW - 1 + half + 1);
    }
    auto issue = [&](int st, int kb) {
        char* t = lds + st * 3 * BLK * ROW;
        tile_dma(a.k1 + koff, a.Sk, kb * BLK, t, threadIdx.x, wave);
        tile_dma(a.k2 + koff, a.Sk, kb * BLK, t + BLK * ROW, threadIdx.x, wave);
        tile_dma(a.v + koff, a.Sk, kb * BLK, t + 2 * BLK * ROW, threadIdx.x, wave);
    };
    if (kb_lo < kb_hi) issue(0, kb_lo);
    for (int kb = kb_lo; kb < kb_hi; ++kb) {
        const int st = (kb - kb_lo) & 1;
        dma_wait_all();   // block kb landed; every wave is done with block kb-1 (the other stage)
        if (kb + 1 < kb_hi) issue(st ^ 1, kb + 1);
        const int kbase = kb * BLK;
        if (q0w >= a.Sq || kbase >= whi || kbase + BLK <= wlo) continue;   // nothing of this block for this wave
        const char* kt = lds + st * 3 * BLK * ROW + br * BLK * ROW;
        const char* vt = lds + st * 3 * BLK * ROW + 2 * BLK * ROW;
        // S^T per 32-key half h: keys 32 h + r(v), query q
        f32x16 s[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int v = 0; v < 16; ++v) s[h][v] = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) s[h] = mfma32(ld_row(kt, 32 * h + c32, 2 * ks + hl), qf[ks], s[h]);
        }
        // mask only blocks that cross a window edge or a sequence end for some query of the wave
        const bool full = q0w + QW <= a.Sq && kbase + BLK <= a.Sk &&
                          (a.window <= 0 || 2 * max(q0w + QW - 1 - kbase, kbase + BLK - 1 - q0w) <= a.window);
        if (!full) {
            const int rel = kbase + 4 * hl - sp.lo;   // key 32 h + r(v), less lo
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const bool ok = (unsigned)(rel + 32 * h + 8 * (v >> 2) + (v & 3)) < (unsigned)sp.n;
                    s[h][v] = ok ? s[h][v] : -INFINITY;
                }
        }
        // block maximum of the raw scores over this lane's 32 keys and the other 32 (lane ^ 32)
        float mx = -INFINITY;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[h][v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(mx > m + kLazy) != 0, 0)) {   // (uniform) a maximum moved far
            const float mn = fmaxf(m, mx);
            const float al = ex2(m - (mn == -INFINITY ? 0.f : mn));   // 0 when m was -inf
            m = mn;
            l *= al;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[db][v] *= al;
        }
        // weights 2^(c s - m), the exponent as one fma of the raw score; m = -inf only while every
        // key so far is invisible, and then every weight is 0. l sums the weights as rounded to
        // bf16, the values the P V product uses (two per dot2 instruction).
        const float base = m == -INFINITY ? 0.f : m;
        bf16x8 p[2][2];   // [half][K step]: values v = 8j .. 8j+7 of the half
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 16; ++v) p[h][v >> 3][v & 7] = (bf16)ex2(__builtin_fmaf(s[h][v], c, -base));
        float ps[2] = {0.f, 0.f};
        const bf16x2 ones = {(bf16)1.f, (bf16)1.f};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ps[e & 1] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p[h][j][2 * e], p[h][j][2 * e + 1]}, ones, ps[e & 1],
                                                                false);
        l += ps[0] + ps[1];
        // O^T += V^T P^T: dims 32 db + lane % 32 (A rows), K step j of half h in the lane's key order
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const int k0 = 32 * h + 16 * j + 4 * hl, n0 = 32 * db + 16 * ((lane >> 4) & 1);
                    o[db] = mfma32(cat44(ld_tr(vt, k0, n0, lane), ld_tr(vt, k0 + 8, n0, lane)), p[h][j], o[db]);
                }
    }
    l += __shfl_xor(l, 32, 64);
    const bool qok = q < a.Sq;
    if (qok && hl == 0) (br ? a.lse2 : a.lse1)[(int64_t)bh * a.Sq + q] = m + log2f(l);
    // normalised branch output; branch 2 hands its fp32 rows to branch 1 through LDS for O = O1 - O2
    const float il = 1.0f / l;
    bf16* ob = (br ? a.o2 : a.o1) + qoff + (int64_t)q * HD;
    constexpr int YS = 68;   // floats per staged row (16-byte aligned, rows 4 banks apart)
    float* y2s = reinterpret_cast<float*>(lds) + (size_t)((wave & 1) * QW + c32) * YS;
    __syncthreads();   // every wave is done with the K/V stages
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
            const int d0 = 32 * db + 8 * vg + 4 * hl;   // dims d0 .. d0+3 = values v = 4 vg .. 4 vg + 3
            float4 y;
            y.x = o[db][4 * vg] * il;
            y.y = o[db][4 * vg + 1] * il;
            y.z = o[db][4 * vg + 2] * il;
            y.w = o[db][4 * vg + 3] * il;
            if (qok) *reinterpret_cast<bf16x4*>(ob + d0) = bf16x4{(bf16)y.x, (bf16)y.y, (bf16)y.z, (bf16)y.w};
            if (br) *reinterpret_cast<float4*>(y2s + d0) = y;
            o[db][4 * vg] = y.x;
            o[db][4 * vg + 1] = y.y;
            o[db][4 * vg + 2] = y.z;
            o[db][4 * vg + 3] = y.w;
        }
    __syncthreads();
    if (br || !qok) return;
    const int b = bh / a.H, hh = bh % a.H;
    bf16* od = a.o + ((int64_t)b * a.Sq + q) * (a.H * HD) + hh * HD;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
            const int d0 = 32 * db + 8 * vg + 4 * hl;
            const float4 y2 = *reinterpret_cast<const float4*>(y2s + d0);
            *reinterpret_cast<bf16x4*>(od + d0) =
                bf16x4{(bf16)(o[db][4 * vg] - y2.x), (bf16)(o[db][4 * vg + 1] - y2.y), (bf16)(o[db][4 * vg + 2] - y2.z),
                       (bf16)(o[db][4 * vg + 3] - y2.w)};
        }
}

// ------------------------------------------------------------------------------------ backward
// Dn_i[bh][q] = sum_d dO[b][q][h][d] * O_i[bh][q][d]; dOh[bh][q][d] = bf16(dO) (head-major).
// Sixteen lanes per (bh, q), 4 dims each (16-byte dO, 8-byte O_i loads), the dot products summed
// over the 16 lanes by group16_sum: the same arithmetic as the epilogue of the product that
// computes dO (the GEMM's attention dO epilogue), which writes these outputs itself where its
// tiles allow.
__global__ __launch_bounds__(kThreads) void attn_bwd_dot_kernel(const float* __restrict__ dO, const bf16* __restrict__ o1,
                                                                const bf16* __restrict__ o2, int BH, int H, int Sq,
                                                                bf16* __restrict__ dOh, float* __restrict__ dn1,
                                                                float* __restrict__ dn2) {
    const unsigned item = (blockIdx.x * kThreads + threadIdx.x) >> 4;
    const int d0 = (threadIdx.x & 15) * 4;
    if (item >= (unsigned)BH * (unsigned)Sq) return;   // uniform over the item's 16 lanes
    const unsigned bh = item / (unsigned)Sq, q = item - bh * (unsigned)Sq;
    const unsigned b = bh / (unsigned)H, h = bh - b * (unsigned)H;
    const float4 x = *reinterpret_cast<const float4*>(dO + ((int64_t)b * Sq + q) * (H * HD) + h * HD + d0);
    const int64_t idx = (int64_t)item * HD + d0;
    const uint2 a1 = *reinterpret_cast<const uint2*>(o1 + idx), a2 = *reinterpret_cast<const uint2*>(o2 + idx);
    const bf16 xo[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
    *reinterpret_cast<uint2*>(dOh + idx) = __builtin_bit_cast(uint2, xo);
    const float s1 = sa3k::group16_sum(sa3k::dot4_bf16(x, a1)), s2 = sa3k::group16_sum(sa3k::dot4_bf16(x, a2));
    if (d0 == 0) {
        dn1[item] = s1;
        dn2[item] = s2;
    }
}

struct BwdArgs {
    const bf16 *q1, *k1, *q2, *k2, *v, *dO;   // [BH][S][64]
    const float *lse1, *lse2, *dn1, *dn2;     // [BH][Sq]
    int Sq, Sk, window;
    float scale;
    float *dq1, *dq2, *dk1, *dk2, *dv;        // [BH][S][64] f32
    // dK/dV with the query blocks of a key block split over qsplit workgroups (blockIdx.z): raw
    // partial sums [qsplit][3 = dV, dK1, dK2][BH][Sk][64] in part, summed by attn_bwd_dkdv_sum
    int qsplit;
    float* part;
};

// Per key block: dK1, dK2, dV. S = Q K^T with lane = key (lane%16), queries 4g+v per 16-query tile.
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv_kernel(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) char lds[2 * 3 * BLK * ROW];   // 2 stages x {Q1, Q2, dO}
    __shared__ __attribute__((aligned(16))) float vec[2][4][BLK];            // lse1, lse2, dn1, dn2
    int kb, bh;
    heavy_first(kb, bh);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, r = lane & 15;
    const int64_t qoff = (int64_t)bh * a.Sq * HD, koff = (int64_t)bh * a.Sk * HD;
    const int key = kb * BLK + w * 16 + r;     // this lane's key
    const float c = a.scale * kLog2e;
    // the queries that see this key: |q - key| <= window/2 and q < Sq (none for a key past Sk)
    const Span qsp = key < a.Sk ? visible(key, a.Sq, a.window) : Span{0, 0};

    bf16x8 k1f[2], k2f[2], vf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        uint4 z = make_uint4(0, 0, 0, 0), u1 = z, u2 = z, u3 = z;
        if (key < a.Sk) {
            u1 = *reinterpret_cast<const uint4*>(a.k1 + koff + (int64_t)key * HD + ks * 32 + g * 8);
            u2 = *reinterpret_cast<const uint4*>(a.k2 + koff + (int64_t)key * HD + ks * 32 + g * 8);
            u3 = *reinterpret_cast<const uint4*>(a.v + koff + (int64_t)key * HD + ks * 32 + g * 8);
        }
        k1f[ks] = __builtin_bit_cast(bf16x8, u1);
        k2f[ks] = __builtin_bit_cast(bf16x8, u2);
        vf[ks] = __builtin_bit_cast(bf16x8, u3);
    }
    f32x4 dvt[4], dk1t[4], dk2t[4];   // transposed accumulators: rows dims dt*16 + 4g + v, col = key
#pragma unroll
    for (int i = 0; i < 4; ++i) dvt[i] = dk1t[i] = dk2t[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    int qb_lo, qb_hi;
    band_range(kb, a.Sq, a.window, qb_lo, qb_hi);
    if (a.qsplit > 1) {   // this workgroup's share of the query blocks
        const int per = (qb_hi - qb_lo + a.qsplit - 1) / a.qsplit;
        qb_lo = min(qb_hi, qb_lo + (int)blockIdx.z * per);
        qb_hi = min(qb_hi, qb_lo + per);
    }
    const int64_t voff = (int64_t)bh * a.Sq;
    auto issue = [&](int st, int qb) {
        char* t = lds + st * 3 * BLK * ROW;
        tile_dma(a.q1 + qoff, a.Sq, qb * BLK, t, threadIdx.x, wave);
        tile_dma(a.q2 + qoff, a.Sq, qb * BLK, t + BLK * ROW, threadIdx.x, wave);
        tile_dma(a.dO + qoff, a.Sq, qb * BLK, t + 2 * BLK * ROW, threadIdx.x, wave);
        if (wave == 0) {
            vec_dma(a.lse1 + voff, a.Sq, qb * BLK, vec[st][0], lane);
            vec_dma(a.lse2 + voff, a.Sq, qb * BLK, vec[st][1], lane);
            vec_dma(a.dn1 + voff, a.Sq, qb * BLK, vec[st][2], lane);
            vec_dma(a.dn2 + voff, a.Sq, qb * BLK, vec[st][3], lane);
        }
    };
    if (qb_lo < qb_hi) issue(0, qb_lo);
    for (int qb = qb_lo; qb < qb_hi; ++qb) {
        const int st = (qb - qb_lo) & 1;
        dma_wait_all();   // block qb landed; every wave is done with block qb-1 (the other stage)
        if (qb + 1 < qb_hi) issue(st ^ 1, qb + 1);
        const char* q1s = lds + st * 3 * BLK * ROW;
        const char* q2s = q1s + BLK * ROW;
        const char* dos = q1s + 2 * BLK * ROW;
        const float* sl1 = vec[st][0];
        const float* sl2 = vec[st][1];
        const float* sd1 = vec[st][2];
        const float* sd2 = vec[st][3];
        // per 16-query tile qt: S1, S2, dP with rows = queries qt*16 + 4g + v, col = key
        const bool full = block_full(qb, kb, a.Sq, a.Sk, a.window);   // block-uniform: no masking
        const int rel = qb * BLK + 4 * g - qsp.lo;   // query qt*16 + 4g + v, less lo, is rel + 16 qt + v
        // one 32-query chunk at a time (fewer live registers): its two 16-query tiles give
        // (P1 - P2), dS1, dS2 as B operands over 8 queries per lane group, then
        // dV^T += dO^T (P1 - P2); dK_i^T += Q_i^T dS_i  (A: transposed tiles)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            bf16x8 pd, ds1, ds2;
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
                const int qt = 2 * ch + qq;
                f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = s1, dp = s1;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    s1 = mfma(ld_row(q1s, qt * 16 + r, ks * 4 + g), k1f[ks], s1);
                    s2 = mfma(ld_row(q2s, qt * 16 + r, ks * 4 + g), k2f[ks], s2);
                    dp = mfma(ld_row(dos, qt * 16 + r, ks * 4 + g), vf[ks], dp);
                }
                if (!full) {   // hidden pairs get score -inf, hence weight 0 and dS 0
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const bool ok = (unsigned)(rel + 16 * qt + v) < (unsigned)qsp.n;
                        s1[v] = ok ? s1[v] : -INFINITY;
                        s2[v] = ok ? s2[v] : -INFINITY;
                    }
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ql = qt * 16 + 4 * g + v;
                    const float p1 = ex2(fmaf(s1[v], c, -sl1[ql]));
                    const float p2 = ex2(fmaf(s2[v], c, -sl2[ql]));
                    const int e = qq * 4 + v;
                    pd[e] = (bf16)(p1 - p2);
                    ds1[e] = (bf16)(p1 * (dp[v] - sd1[ql]));
                    ds2[e] = (bf16)(-p2 * (dp[v] - sd2[ql]));
                }
            }
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int c0 = 32 * ch + 4 * g, c1 = 32 * ch + 16 + 4 * g;
                dvt[dt] = mfma(cat44(ld_tr(dos, c0, dt * 16, lane), ld_tr(dos, c1, dt * 16, lane)), pd, dvt[dt]);
                dk1t[dt] = mfma(cat44(ld_tr(q1s, c0, dt * 16, lane), ld_tr(q1s, c1, dt * 16, lane)), ds1, dk1t[dt]);
                dk2t[dt] = mfma(cat44(ld_tr(q2s, c0, dt * 16, lane), ld_tr(q2s, c1, dt * 16, lane)), ds2, dk2t[dt]);
            }
        }
    }
    if (key >= a.Sk) return;
    if (a.qsplit > 1) {
        const int64_t plane = (int64_t)gridDim.y * a.Sk * HD;
        float* pz = a.part + (int64_t)blockIdx.z * 3 * plane;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t idx = koff + (int64_t)key * HD + dt * 16 + 4 * g + v;
                pz[idx] = dvt[dt][v];
                pz[plane + idx] = dk1t[dt][v];
                pz[2 * plane + idx] = dk2t[dt][v];
            }
        return;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t idx = koff + (int64_t)key * HD + dt * 16 + 4 * g + v;
            a.dv[idx] = dvt[dt][v];
            a.dk1[idx] = a.scale * dk1t[dt][v];
            a.dk2[idx] = a.scale * dk2t[dt][v];
        }
}

// dV, dK1, dK2 from the query-split partials, summed in split order (4 values per thread)
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv_sum(BwdArgs a, int64_t plane) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i >= plane) return;
    float4 s[3];
#pragma unroll
    for (int o = 0; o < 3; ++o) s[o] = make_float4(0.f, 0.f, 0.f, 0.f);
    // four splits' partials loaded per memory round trip (indices past the last split re-read it and
    // are not added); the sums are added in split order from zero
    for (int z = 0; z < a.qsplit; z += 4) {
        float4 v[4][3];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int o = 0; o < 3; ++o)
                v[k][o] = *reinterpret_cast<const float4*>(a.part + ((int64_t)min(z + k, a.qsplit - 1) * 3 + o) * plane + i);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (z + k < a.qsplit)
#pragma unroll
                for (int o = 0; o < 3; ++o)
                    s[o] = make_float4(s[o].x + v[k][o].x, s[o].y + v[k][o].y, s[o].z + v[k][o].z, s[o].w + v[k][o].w);
    }
    *reinterpret_cast<float4*>(a.dv + i) = s[0];
    *reinterpret_cast<float4*>(a.dk1 + i) = make_float4(a.scale * s[1].x, a.scale * s[1].y, a.scale * s[1].z, a.scale * s[1].w);
    *reinterpret_cast<float4*>(a.dk2 + i) = make_float4(a.scale * s[2].x, a.scale * s[2].y, a.scale * s[2].z, a.scale * s[2].w);
}

// Per query block: dQ1, dQ2. S^T = K Q^T (lane = query), dP^T = V dO^T.
__global__ __launch_bounds__(kThreads) void attn_bwd_dq_kernel(BwdArgs a) {
    __shared__ __attribute__((aligned(1024))) char lds[2 * 3 * BLK * ROW];   // 2 stages x {K1, K2, V}
    int qb, bh;
    heavy_first(qb, bh);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, r = lane & 15;
    const int64_t qoff = (int64_t)bh * a.Sq * HD, koff = (int64_t)bh * a.Sk * HD;
    const int qrow = qb * BLK + w * 16 + r;
    const float c = a.scale * kLog2e;

    bf16x8 q1f[2], q2f[2], dof[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        uint4 z = make_uint4(0, 0, 0, 0), u1 = z, u2 = z, u3 = z;
        if (qrow < a.Sq) {
            u1 = *reinterpret_cast<const uint4*>(a.q1 + qoff + (int64_t)qrow * HD + ks * 32 + g * 8);
            u2 = *reinterpret_cast<const uint4*>(a.q2 + qoff + (int64_t)qrow * HD + ks * 32 + g * 8);
            u3 = *reinterpret_cast<const uint4*>(a.dO + qoff + (int64_t)qrow * HD + ks * 32 + g * 8);
        }
        q1f[ks] = __builtin_bit_cast(bf16x8, u1);
        q2f[ks] = __builtin_bit_cast(bf16x8, u2);
        dof[ks] = __builtin_bit_cast(bf16x8, u3);
    }
    const bool qok = qrow < a.Sq;
    const Span sp = qok ? visible(qrow, a.Sk, a.window) : Span{0, 0};   // keys this query sees
    const float L1 = qok ? a.lse1[(int64_t)bh * a.Sq + qrow] : 0.f;
    const float L2 = qok ? a.lse2[(int64_t)bh * a.Sq + qrow] : 0.f;
    const float D1 = qok ? a.dn1[(int64_t)bh * a.Sq + qrow] : 0.f;
    const float D2 = qok ? a.dn2[(int64_t)bh * a.Sq + qrow] : 0.f;
    f32x4 dq1[4], dq2[4];   // rows queries 4g+v, col dims dt*16 + r
#pragma unroll
    for (int i = 0; i < 4; ++i) dq1[i] = dq2[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    int kb_lo, kb_hi;
    band_range(qb, a.Sk, a.window, kb_lo, kb_hi);
    auto issue = [&](int st, int kb) {
        char* t = lds + st * 3 * BLK * ROW;
        tile_dma(a.k1 + koff, a.Sk, kb * BLK, t, threadIdx.x, wave);
        tile_dma(a.k2 + koff, a.Sk, kb * BLK, t + BLK * ROW, threadIdx.x, wave);
        tile_dma(a.v + koff, a.Sk, kb * BLK, t + 2 * BLK * ROW, threadIdx.x, wave);
    };
    if (kb_lo < kb_hi) issue(0, kb_lo);
    for (int kb = kb_lo; kb < kb_hi; ++kb) {
        const int st = (kb - kb_lo) & 1;
        dma_wait_all();   // block kb landed; every wave is done with block kb-1 (the other stage)
        if (kb + 1 < kb_hi) issue(st ^ 1, kb + 1);
        const char* k1s = lds + st * 3 * BLK * ROW;
        const char* k2s = k1s + BLK * ROW;
        const char* vs = k1s + 2 * BLK * ROW;
        bf16x8 ds1[2], ds2[2];
        const bool full = block_full(qb, kb, a.Sq, a.Sk, a.window);   // block-uniform: no masking
        const int rel = kb * BLK + 4 * g - sp.lo;   // key kt*16 + 4g + v, less lo, is rel + 16 kt + v
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = s1, dp = s1;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                s1 = mfma(ld_row(k1s, kt * 16 + r, ks * 4 + g), q1f[ks], s1);
                s2 = mfma(ld_row(k2s, kt * 16 + r, ks * 4 + g), q2f[ks], s2);
                dp = mfma(ld_row(vs, kt * 16 + r, ks * 4 + g), dof[ks], dp);
            }
            if (!full) {   // hidden pairs get score -inf, hence weight 0 and dS 0
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const bool ok = (unsigned)(rel + 16 * kt + v) < (unsigned)sp.n;
                    s1[v] = ok ? s1[v] : -INFINITY;
                    s2[v] = ok ? s2[v] : -INFINITY;
                }
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float p1 = ex2(fmaf(s1[v], c, -L1));
                const float p2 = ex2(fmaf(s2[v], c, -L2));
                const int e = (kt & 1) * 4 + v;
                ds1[kt >> 1][e] = (bf16)(p1 * (dp[v] - D1));
                ds2[kt >> 1][e] = (bf16)(-p2 * (dp[v] - D2));
            }
        }
        // dQ_i += dS_i K_i: B = K^T tile rows = dims, 8 keys per lane group
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int c0 = 32 * ch + 4 * g, c1 = 32 * ch + 16 + 4 * g;
                dq1[dt] = mfma(ds1[ch], cat44(ld_tr(k1s, c0, dt * 16, lane), ld_tr(k1s, c1, dt * 16, lane)), dq1[dt]);
                dq2[dt] = mfma(ds2[ch], cat44(ld_tr(k2s, c0, dt * 16, lane), ld_tr(k2s, c1, dt * 16, lane)), dq2[dt]);
            }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int q = qb * BLK + w * 16 + 4 * g + v;
        if (q >= a.Sq) continue;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int64_t idx = qoff + (int64_t)q * HD + dt * 16 + r;
            a.dq1[idx] = a.scale * dq1[dt][v];
            a.dq2[idx] = a.scale * dq2[dt][v];
        }
    }
}

}  // namespace

// ------------------------------------------------------------------------------------ host
namespace sa3k {

void attn_forward(sa3k_ctx* ctx, const bf16* q1, const bf16* k1, const bf16* q2, const bf16* k2, const bf16* v,
                  int B, int H, int Sq, int Sk, int window, float scale, bf16* o, bf16* o1, bf16* o2,
                  float* lse1, float* lse2) {
    SA3K_REQUIRE(B > 0 && H > 0 && Sq > 0 && Sk > 0, "attention extents must be positive");
    SA3K_REQUIRE(window == 0 || Sq == Sk, "a window needs self-attention (Sq == Sk)");
    FwdArgs a{q1, k1, q2, k2, v, H, Sq, Sk, window, scale, o, o1, o2, lse1, lse2};
    KernelScope ks(ctx, Sq == Sk ? "attn_fwd" : "attn_fwd_cross");
    // the branch-per-wave kernel pays a longer prologue and epilogue per workgroup and wins from
    // about three key blocks per workgroup on (self-attention); short key sequences keep the other
    if (ctx->attn_fwd32 && scale > 0.f && Sk > 2 * BLK) {
        launch_k(ctx, true, attn_fwd32_kernel, dim3((unsigned)ceil_div(Sq, BLK), (unsigned)(B * H)), dim3(kThreads),
                 0, a);
    } else {
        launch_k(ctx, true, attn_fwd_kernel, dim3((unsigned)ceil_div(Sq, BLK), (unsigned)(B * H)), dim3(kThreads), 0, a);
    }
    SA3K_LAUNCHED();
}

// dO: f32 [B][Sq][H*64] token-major; scratch dOh bf16 [BH][Sq][64], dn1/dn2 f32 [BH][Sq]
void attn_backward(sa3k_ctx* ctx, const bf16* q1, const bf16* k1, const bf16* q2, const bf16* k2, const bf16* v,
                   const bf16* o1, const bf16* o2, const float* lse1, const float* lse2, const float* dO,
                   int B, int H, int Sq, int Sk, int window, float scale, bf16* dOh, float* dn1, float* dn2,
                   float* dq1, float* dk1, float* dq2, float* dk2, float* dv, bool dot_done) {
    SA3K_REQUIRE(window == 0 || Sq == Sk, "a window needs self-attention (Sq == Sk)");
    const int BH = B * H;
    // dQ (third stream) and dK/dV (main stream) only share inputs: they run side by side once the
    // row dots are done (the dot kernel records the fork event). dot_done: the product that
    // computed dO has written dOh and the row dots (dO itself is not read).
    const bool side = side_usable(ctx);
    if (!dot_done) {
        if (side) fork_arm(ctx);
        KernelScope ks(ctx, Sq == Sk ? "attn_bwd_dot" : "attn_bwd_dot_cross");
        const int64_t items = (int64_t)BH * Sq;
        SA3K_REQUIRE(items * 16 < ((int64_t)1 << 32), "too many (batch, head, query) rows for one attention call");
        launch_k(ctx, true, attn_bwd_dot_kernel, dim3((unsigned)ceil_div(items * 16, kThreads)), dim3(kThreads), 0,
                 dO, o1, o2, BH, H, Sq, dOh, dn1, dn2);
        SA3K_LAUNCHED();
    }
    BwdArgs a{q1, k1, q2, k2, v, dOh, lse1, lse2, dn1, dn2, Sq, Sk, window, scale, dq1, dq2, dk1, dk2, dv, 1, nullptr};
    // Few key blocks (cross-attention to a short context): split every key block's query range
    // over several workgroups so the grid fills the chip, then sum the partials.
    const int nkb = (int)ceil_div(Sk, BLK), nqb = (int)ceil_div(Sq, BLK);
    const int64_t plane = (int64_t)BH * Sk * HD;
    if (window == 0 && (int64_t)nkb * BH < 512) {
        a.qsplit = (int)std::min<int64_t>({(int64_t)nqb, 16, ceil_div(512, (int64_t)nkb * BH)});
        if (a.qsplit > 1) a.part = gemm_workspace_bytes(ctx, (size_t)a.qsplit * 3 * plane * sizeof(float));
    }
    if (side) quick_fork(ctx);
    {
        OnQuick os(ctx, side);
        KernelScope ks(ctx, Sq == Sk ? "attn_bwd_dq" : "attn_bwd_dq_cross");
        attn_bwd_dq_kernel<<<dim3((unsigned)ceil_div(Sq, BLK), (unsigned)BH), kThreads, 0, ctx->stream>>>(a);
        SA3K_LAUNCHED();
    }
    {
        KernelScope ks(ctx, Sq == Sk ? "attn_bwd_dkdv" : "attn_bwd_dkdv_cross");
        attn_bwd_dkdv_kernel<<<dim3((unsigned)nkb, (unsigned)BH, (unsigned)a.qsplit), kThreads, 0, ctx->stream>>>(a);
        SA3K_LAUNCHED();
        if (a.qsplit > 1) {
            attn_bwd_dkdv_sum<<<(unsigned)ceil_div(plane / 4, kThreads), kThreads, 0, ctx->stream>>>(a, plane);
            SA3K_LAUNCHED();
        }
    }
    if (side) quick_join(ctx);   // the callers consume dQ next
}

}  // namespace sa3k

// ------------------------------------------------------------------------------------ C ABI
extern "C" {

SA3K_API int sa3k_diff_attn_fwd(sa3k_ctx* ctx, const void* q1, const void* k1, const void* q2, const void* k2,
                                const void* v, int B, int H, int Sq, int Sk, int head_dim, int window, float scale,
                                void* o, void* o1, void* o2, float* lse1, float* lse2) {
    return sa3k_guard(ctx, "sa3k_diff_attn_fwd", [&] {
        SA3K_REQUIRE(head_dim == HD, "head_dim must be 64");
        SA3K_REQUIRE(q1 && k1 && q2 && k2 && v && o && o1 && o2 && lse1 && lse2, "null pointer");
        sa3k::attn_forward(ctx, (const bf16*)q1, (const bf16*)k1, (const bf16*)q2, (const bf16*)k2, (const bf16*)v,
                           B, H, Sq, Sk, window, scale, (bf16*)o, (bf16*)o1, (bf16*)o2, lse1, lse2);
    });
}

SA3K_API int sa3k_diff_attn_bwd(sa3k_ctx* ctx, const void* q1, const void* k1, const void* q2, const void* k2,
                                const void* v, const void* o1, const void* o2, const float* lse1, const float* lse2,
                                const float* dO, int B, int H, int Sq, int Sk, int head_dim, int window, float scale,
                                void* scratch_dOh, float* scratch_dn, float* dq1, float* dk1, float* dq2, float* dk2,
                                float* dv) {
    return sa3k_guard(ctx, "sa3k_diff_attn_bwd", [&] {
        SA3K_REQUIRE(head_dim == HD, "head_dim must be 64");
        SA3K_REQUIRE(q1 && k1 && q2 && k2 && v && o1 && o2 && lse1 && lse2 && dO && scratch_dOh && scratch_dn,
                     "null pointer");
        SA3K_REQUIRE(dq1 && dk1 && dq2 && dk2 && dv, "null gradient pointer");
        const int64_t n = (int64_t)B * H * Sq;
        sa3k::attn_backward(ctx, (const bf16*)q1, (const bf16*)k1, (const bf16*)q2, (const bf16*)k2, (const bf16*)v,
                            (const bf16*)o1, (const bf16*)o2, lse1, lse2, dO, B, H, Sq, Sk, window, scale,
                            (bf16*)scratch_dOh, scratch_dn, scratch_dn + n, dq1, dk1, dq2, dk2, dv, false);
    });
}

}  // extern "C"
