// K1/K2 fast path: C = A . B^T with both operands already in the compute type (bf16 or f32).
//
// Operand tiles go straight from global memory into LDS with global_load_lds_dwordx4 (gfx950),
// so no VGPR staging and no per-element work happens in the K loop: the loop is DMA issue,
// one barrier, and 16-byte LDS fragment reads feeding the MFMAs. A STAGES-deep LDS ring keeps
// STAGES-1 K tiles in flight. LDS rows are 128 bytes (64 bf16 / 32 f32 of K) without padding;
// the eight 16-byte chunks of row r are stored XOR-swizzled (chunk kc at kc ^ swz(r)) so that the
// rows a fragment read touches fall into distinct banks. The DMA writes 64 consecutive 16-byte
// slots per wave instruction, so the swizzle is applied on the global side: the lane that owns
// LDS slot s fetches the chunk that belongs there.
//
// Rows past M+Mx / N are clamped to a valid row (their results are never stored); K chunks past
// K2 in the second segment read a zero page, since they feed valid outputs.
#include "gemm.h"
#include "headprep.h"

#include <algorithm>

namespace sa3k {

struct DmaParams {
    const void* A; int64_t lda;
    const void* B; int64_t ldb;
    const void* A2; int64_t lda2;
    const void* B2; int64_t ldb2;
    int K2;
    int64_t M, N, K;
    float alpha;
    const float* colscale;
    const float* bias;
    float* C; int64_t ldc; int accumulate;
    bf16* Cb; int64_t ldcb;
    float* U; bf16* Ub; int64_t ldu;
    int64_t Mx;
    const void* Ax; int64_t ldax;
    const void* A2x; int64_t lda2x;
    float* Cx; int64_t ldcx; int accumulate_x;
    bf16* Cbx;
    float* ws;
    int kps;
    const void* zero;   // >= 16 zero bytes
    int* counters;      // split-K arrival counters per tile (all zero between launches), or null
    // byte extents of A, Ax and B as read by the main segment: set (non-zero) when each fits the
    // 32-bit offsets of a buffer descriptor, which then carries the main-segment loads
    uint32_t a_bytes, ax_bytes, b_bytes;
    int vec_epi;   // outputs allow the 16-byte staged epilogue (aligned rows, N % 4 == 0)
    int nt_store;  // staged-epilogue output stores are non-temporal
    int prescale;  // colscale applied to the main segment in the K loop, not in the epilogue
    // extra columns (GemmDesc::Nx): B rows N .. Nt-1 come from Bx; Nt = N + Nx
    int64_t Nx, Nt;
    const void* Bx; int64_t ldbx;
    float alpha_x;
    bf16* Cbn; int64_t ldcn;
    uint32_t bx_bytes;
    int b_kn;   // B stored [K][ldb], N contiguous (GemmDesc::b_kn)
    // main-segment B decoded on its way from LDS into the MFMA operands: bq 1 f16 elements, 2 Q8_0
    // (int8 quants, ldb bytes per row, and f16 block scales Bs, ldbs per row); 0 bf16
    int bq;
    const void* Bs; int64_t ldbs;
    uint32_t bs_bytes;
    // paired SwiGLU epilogue (GemmDesc::sw_*): 256-column tiles below 2 sw_half hold columns
    // [128 t, 128 t + 128) of both halves; 0: off
    int64_t sw_half;
    bf16* sw_g; int64_t sw_ldg;
    int* sw_done;   // host-side: set to 1 by the launcher that keeps the pairing
    HeadPrep hp;    // per-head q/k preparation (GemmDesc::hp), head-prep instantiations only
    int* hp_done;   // host-side, like sw_done
    int c_unfused_only;   // host-side (GemmDesc::c_unfused_only)
    int prio;             // raise the wave priority over the MFMA clusters of the K loop
    AttnDot ad;           // the attention dO epilogue (GemmDesc::ad; doh null: off)
    SwiBwd sb;            // the SwiGLU backward epilogue (GemmDesc::sb; du null: off)
    int* bwd_done;        // host-side, like sw_done
};

namespace {

constexpr int kThreads = 256;
constexpr int kRow = 128;   // LDS bytes per tile row

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// XOR swizzle of the eight 16-byte chunks of a 128-byte LDS row. MFMA operand reads (lane l reads
// chunk 2s + l/32 of row l%32, or chunk 4s + l/16 of row l%16) are bank-conflict-free with it on
// gfx950: rows r and r^1 sit in different bank halves, and the chunk XOR is a bit permutation of
// (r>>1)&7 such that every group of lanes the LDS serves in one pass covers each bank once (the
// previous (r&7)^(r>>3&1) left 2-way conflicts: 3.2 extra cycles per ds_read_b128 on the
// SQ_LDS_BANK_CONFLICT counter). The transposed reads of a [K][N] B operand (ld_tr) still meet
// 2-way conflicts (2 extra cycles per read); the linear map (a2, a1^a2, a0) of a = (r>>1)&7 serves
// them in one pass too, but measured no faster on these kernels (the 128 x 256 products without
// transposed reads 1-2% slower, the [K][N] ones within 1%), so the permutation stays.
__device__ __forceinline__ int swz(int r) {
    const int a = (r >> 1) & 7;
    return (a & 1) | ((a & 2) << 1) | ((a & 4) >> 1);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef short v4s __attribute__((ext_vector_type(4)));

// B operand stored [K][N] (b_kn): a stage's B region holds BN/64 sub-tiles of [64 k][64 n] bf16,
// 128-byte rows with the chunk swizzle above. ld_tr reads them transposed (ds_read_b64_tr_b16):
// every 16-lane group returns, in lane j of the group, T[k0 .. k0+3][n0 + j] of a sub-tile (lane
// j addresses row k0 + j/4, columns n0 + 4 (j%4) .. +3); k0, n0 may differ between the groups.
__device__ __forceinline__ bf16x4 ld_tr(const char* t, int k0, int n0, int lane) {
    const int j = lane & 15, row = k0 + (j >> 2), n = n0 + 4 * (j & 3);
    const char* a = t + row * kRow + (((n >> 3) ^ swz(row)) << 4) + (n & 7) * 2;
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                          (__attribute__((address_space(3))) v4s*)((lds_ptr_t)a)));
}
__device__ __forceinline__ bf16x8 cat44(bf16x4 a, bf16x4 b) {
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Raw buffer descriptor over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const unsigned long long a = (unsigned long long)(uintptr_t)base;
    u32x4 r;
    r.x = (unsigned)a;
    r.y = (unsigned)(a >> 32) & 0xffffu;   // stride 0
    r.z = bytes;                           // num_records
    r.w = 0x00020000u;                     // 32-bit data format, no swizzle
    return r;
}

// Every lane fetches 16 bytes at descriptor offset voff + soff into LDS at lds_addr + lane*16
// (buffer_load ... lds). Measured on MI355X, these overlap with the MFMA stream far better
// than global_load_lds (1.11 vs 0.67 PFLOP/s for the same loop); inline asm for the reason given
// at dma16.
__device__ __forceinline__ void dma16b(const u32x4& rsrc, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds_addr), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory");
}

// 4 bytes per lane into LDS at lds_addr + 4 lane
__device__ __forceinline__ void dma4b(const u32x4& rsrc, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds_addr), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory");
}

// one of two descriptors on a wave-uniform condition, kept in scalar registers
__device__ __forceinline__ u32x4 pick_rsrc(bool c, const u32x4& a, const u32x4& b) {
    const bool u = __builtin_amdgcn_readfirstlane((int)c) != 0;
    u32x4 r;
    r.x = __builtin_amdgcn_readfirstlane(u ? a.x : b.x);
    r.y = __builtin_amdgcn_readfirstlane(u ? a.y : b.y);
    r.z = __builtin_amdgcn_readfirstlane(u ? a.z : b.z);
    r.w = __builtin_amdgcn_readfirstlane(u ? a.w : b.w);
    return r;
}

template <int N>
struct IC {
    static constexpr int value = N;
};
// f(IC<0>{}), ..., f(IC<N-1>{}) in order
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(IC<I>{});
        static_for<N, I + 1>(f);
    }
}

// s_waitcnt vmcnt(n) leaving the other counters untouched (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Every lane fetches 16 bytes from g into LDS at lds_addr + lane*16 (lds_addr wave-uniform). Issued as inline
// asm, so the compiler does not see an LDS write it must order against the MFMA operand reads:
// its wait insertion cannot tell the stage being filled from the stages being read once the K loop
// wraps, and would drain every DMA (vmcnt 0) before each read. The kernel orders them itself
// (vmcnt waits + barrier per K step). M0 holds the LDS base and is written right before each use;
// nothing else in these kernels keeps a value in M0.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(g) : "memory");
}

__device__ inline void epilogue_elem(const DmaParams& p, int64_t m, int64_t n, float acc) {
    if (n >= p.N) {   // extra column
        if (m < p.M) p.Cbn[m * p.ldcn + (n - p.N)] = (bf16)(p.alpha_x * acc);
        return;
    }
    float x = p.alpha * acc;
    if (m >= p.M) {
        if (p.Cbx) {
            p.Cbx[(m - p.M) * p.ldcx + n] = (bf16)x;
            return;
        }
        float* cx = p.Cx + (m - p.M) * p.ldcx + n;
        *cx = p.accumulate_x ? *cx + x : x;
        return;
    }
    if (p.U) p.U[m * p.ldu + n] = x;
    if (p.Ub) p.Ub[m * p.ldu + n] = (bf16)x;
    if (p.colscale && !p.prescale) x = x * p.colscale[n];
    if (p.bias) x = x + p.bias[n];
    if (p.C) {
        if (p.accumulate) p.C[m * p.ldc + n] += x;
        else p.C[m * p.ldc + n] = x;
    }
    if (p.Cb) p.Cb[m * p.ldcb + n] = (bf16)x;
}

// Output stores of the staged epilogue, optionally non-temporal (context option gemm_nt_store): the
// output stream (tens of MB per launch) then does not evict the operand lines the other tiles of the
// launch still reuse from L2.
typedef float f32v4 __attribute__((ext_vector_type(4)));
typedef unsigned u32v2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_out(bool nt, float4* p, float4 v) {
    if (nt) __builtin_nontemporal_store(f32v4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32v4*>(p));
    else *p = v;
}
__device__ __forceinline__ void st_out(bool nt, uint2* p, uint2 v) {
    if (nt) __builtin_nontemporal_store(u32v2{v.x, v.y}, reinterpret_cast<u32v2*>(p));
    else *p = v;
}

// Column factors of four consecutive main columns n..n+3 (colscale where the epilogue applies it,
// bias; 1 and 0 otherwise or past N). The staged epilogue loads them once per thread: a thread's
// columns stay the same over every row it stores.
struct EpiCols {
    float4 cs, bs;
};
__device__ inline EpiCols epi_cols(const DmaParams& p, int64_t n) {
    EpiCols k{make_float4(1.0f, 1.0f, 1.0f, 1.0f), make_float4(0.0f, 0.0f, 0.0f, 0.0f)};
    if (n < p.N) {
        if (p.colscale && !p.prescale) k.cs = *reinterpret_cast<const float4*>(p.colscale + n);
        if (p.bias) k.bs = *reinterpret_cast<const float4*>(p.bias + n);
    }
    return k;
}
// Wait for the loads of k here, ahead of the output stores. A use of k after stores were issued
// would wait on the vector-memory counter, which the stores count too (in order), so every row's
// epilogue would wait for the previous row's stores to complete.
__device__ __forceinline__ void epi_cols_ready(const EpiCols& k) {
    asm volatile("" ::"v"(k.cs.x), "v"(k.cs.y), "v"(k.cs.z), "v"(k.cs.w), "v"(k.bs.x), "v"(k.bs.y), "v"(k.bs.z),
                 "v"(k.bs.w));
}
// colscale, then bias, on x = alpha (A B^T + ...) of main rows
__device__ inline float4 epi_scale(const DmaParams& p, float4 x, const EpiCols& k) {
    if (p.colscale && !p.prescale) x = make_float4(x.x * k.cs.x, x.y * k.cs.y, x.z * k.cs.z, x.w * k.cs.w);
    if (p.bias) x = make_float4(x.x + k.bs.x, x.y + k.bs.y, x.z + k.bs.z, x.w + k.bs.w);
    return x;
}

// Epilogue of four consecutive columns n..n+3 of row m (host-checked: 16-byte aligned rows, N a
// multiple of 4), same operations and order as epilogue_elem; k = epi_cols(p, n). Returns the
// main-row value before accumulation into C (unspecified for extra rows and columns).
__device__ inline float4 epilogue_vec4(const DmaParams& p, int64_t m, int64_t n, float4 a, const EpiCols& k) {
    if (n >= p.N) {   // four extra columns (N % 4 == 0)
        if (m < p.M) {
            const bf16 b[4] = {(bf16)(p.alpha_x * a.x), (bf16)(p.alpha_x * a.y), (bf16)(p.alpha_x * a.z),
                               (bf16)(p.alpha_x * a.w)};
            *reinterpret_cast<uint2*>(p.Cbn + m * p.ldcn + (n - p.N)) = __builtin_bit_cast(uint2, b);
        }
        return a;
    }
    float4 x = make_float4(p.alpha * a.x, p.alpha * a.y, p.alpha * a.z, p.alpha * a.w);
    if (m >= p.M) {
        if (p.Cbx) {
            bf16 b[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
            *reinterpret_cast<uint2*>(p.Cbx + (m - p.M) * p.ldcx + n) = __builtin_bit_cast(uint2, b);
            return x;
        }
        float4* cx = reinterpret_cast<float4*>(p.Cx + (m - p.M) * p.ldcx + n);
        if (p.accumulate_x) {
            const float4 o = *cx;
            x = make_float4(o.x + x.x, o.y + x.y, o.z + x.z, o.w + x.w);
        }
        *cx = x;
        return x;
    }
    if (p.U) st_out(p.nt_store, reinterpret_cast<float4*>(p.U + m * p.ldu + n), x);
    if (p.Ub) {
        bf16 b[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
        st_out(p.nt_store, reinterpret_cast<uint2*>(p.Ub + m * p.ldu + n), __builtin_bit_cast(uint2, b));
    }
    x = epi_scale(p, x, k);
    const float4 v = x;
    if (p.C) {
        float4* c = reinterpret_cast<float4*>(p.C + m * p.ldc + n);
        if (p.accumulate) {
            const float4 o = *c;
            x = make_float4(o.x + x.x, o.y + x.y, o.z + x.z, o.w + x.w);
        }
        st_out(p.nt_store, c, x);
    }
    if (p.Cb) {
        bf16 b[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
        st_out(p.nt_store, reinterpret_cast<uint2*>(p.Cb + m * p.ldcb + n), __builtin_bit_cast(uint2, b));
    }
    return v;
}
__device__ inline void epilogue_vec4(const DmaParams& p, int64_t m, int64_t n, float4 a) {
    epilogue_vec4(p, m, n, a, epi_cols(p, n));
}

// Output column of local column c of the 256-column tile tn: with the paired SwiGLU epilogue,
// columns [0, 128) of a tile below 2 sw_half are val columns 128 tn + c and [128, 256) the matching
// glu columns sw_half + 128 tn + c - 128; otherwise (and for the extra-column tile past 2 sw_half)
// 256 tn + c.
__device__ __forceinline__ int64_t tile_col(const DmaParams& p, int64_t n0, int c) {
    if (p.sw_half > 0 && n0 < 2 * p.sw_half) {
        const int64_t h0 = n0 >> 1;
        return c < 128 ? h0 + c : p.sw_half + h0 + (c - 128);
    }
    return n0 + c;
}

// tile_col for a tile BN columns wide: only 256-column tiles are ever paired
template <int BN>
__device__ __forceinline__ int64_t tile_col_bn(const DmaParams& p, int64_t n0, int c) {
    if constexpr (BN == 256) return tile_col(p, n0, c);
    else return n0 + c;
}

__device__ __forceinline__ void st_out(bool nt, unsigned* p, unsigned v) {
    if (nt) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// Paired SwiGLU tile (GemmDesc::sw_half): lane l < 32 of a wave holds the val chunk (columns nv ..
// nv + 3) of its row's epilogue value, lane l + 32 the glu chunk (sw_half + nv ..); the two swap
// values and each writes two of the four g = bf16(val * glu * sigmoid(glu)), the lower lane columns
// nv, nv + 1, the upper one nv + 2, nv + 3 (at gp). Called by all 64 lanes of a wave with one row.
__device__ inline void swiglu_pair_store(const DmaParams& p, bf16* gp, bool lo, float4 mine) {
    float4 other;
    other.x = __shfl_xor(mine.x, 32);
    other.y = __shfl_xor(mine.y, 32);
    other.z = __shfl_xor(mine.z, 32);
    other.w = __shfl_xor(mine.w, 32);
    const float4 v = lo ? mine : other, u = lo ? other : mine;
    const float v0 = lo ? v.x : v.z, v1 = lo ? v.y : v.w, u0 = lo ? u.x : u.z, u1 = lo ? u.y : u.w;
    const bf16 o[2] = {(bf16)(v0 * u0 * swiglu_sigmoid(u0)), (bf16)(v1 * u1 * swiglu_sigmoid(u1))};
    st_out(p.nt_store, reinterpret_cast<unsigned*>(gp), __builtin_bit_cast(unsigned, o));
}

// Main-row, main-column outputs of one staged-epilogue thread, addressed by per-lane pointers at
// the thread's first row of a pass; a later row adds a wave-uniform row offset (no per-row 64-bit
// index products, and the output bases and strides do not stay live in scalar registers).
struct EpiRow {
    float* C; bf16* Cb; float* U; bf16* Ub;
};
__device__ inline EpiRow epi_row(const DmaParams& p, int64_t m, int64_t n) {
    EpiRow r;
    r.C = p.C ? p.C + m * p.ldc + n : nullptr;
    r.Cb = p.Cb ? p.Cb + m * p.ldcb + n : nullptr;
    r.U = p.U ? p.U + m * p.ldu + n : nullptr;
    r.Ub = p.Ub ? p.Ub + m * p.ldu + n : nullptr;
    return r;
}
// epilogue_vec4 for a main row and main columns, dr rows past the pointers of r; returns the value
// before accumulation into C
__device__ inline float4 epilogue_main4(const DmaParams& p, const EpiRow& r, int dr, float4 a, const EpiCols& k) {
    float4 x = make_float4(p.alpha * a.x, p.alpha * a.y, p.alpha * a.z, p.alpha * a.w);
    if (r.U) st_out(p.nt_store, reinterpret_cast<float4*>(r.U + (int64_t)dr * p.ldu), x);
    if (r.Ub) {
        bf16 b[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
        st_out(p.nt_store, reinterpret_cast<uint2*>(r.Ub + (int64_t)dr * p.ldu), __builtin_bit_cast(uint2, b));
    }
    x = epi_scale(p, x, k);
    const float4 v = x;
    if (r.C) {
        float4* c = reinterpret_cast<float4*>(r.C + (int64_t)dr * p.ldc);
        if (p.accumulate) {
            const float4 o = *c;
            x = make_float4(o.x + x.x, o.y + x.y, o.z + x.z, o.w + x.w);
        }
        st_out(p.nt_store, c, x);
    }
    if (r.Cb) {
        bf16 b[4] = {(bf16)x.x, (bf16)x.y, (bf16)x.z, (bf16)x.w};
        st_out(p.nt_store, reinterpret_cast<uint2*>(r.Cb + (int64_t)dr * p.ldcb), __builtin_bit_cast(uint2, b));
    }
    return v;
}

// NW wave64s per workgroup (4 or 8): WMW of them along M, NW/WMW along N, each owning a
// (BM/WMW) x (BN/(NW/WMW)) block of the tile. With 8 waves two share each SIMD, so one wave's
// LDS reads and waits overlap the other's MFMAs inside a single workgroup.
// Q8_0 B tile in LDS (BQ 2): BN rows of 64 quant bytes (four 16-byte chunks, XOR-swizzled by
// qswz), then the rows' two f16 block scales (4 bytes per row, NW x 64 slots), then a dummy area for
// the loads that pad a tile's DMA count to the bf16 tile's (so the ring's vmcnt accounting holds).
__device__ __forceinline__ int qswz(int r) { return (r >> 1) & 3; }

// Output stores of the per-head q/k preparation: row m, output column nq (a multiple of 4 below N)
// with its 16-lane head group; k the tile's part; tab_row the token's RoPE table row (LDS).
struct HeadPrepLane {
    int k;                // part of the tile's columns
    const float* gamma;   // part k's gain (null: copied)
    bf16* out;            // part k's head-major output
    bool rope;
    float4 g;             // this lane's four gains
};
__device__ inline HeadPrepLane head_prep_lane(const DmaParams& p, int64_t n0, int64_t nq) {
    HeadPrepLane l{(int)(n0 / p.hp.dim), nullptr, nullptr, false, make_float4(0.f, 0.f, 0.f, 0.f)};
#pragma unroll
    for (int i = 0; i < 5; ++i)   // selects, no dynamic index into the kernel arguments
        if (i == l.k) {
            l.gamma = p.hp.gamma[i];
            l.out = p.hp.out[i];
            l.rope = p.hp.rope[i] != 0 && p.hp.gamma[i] != nullptr;
        }
    if (l.gamma) l.g = *reinterpret_cast<const float4*>(l.gamma + (nq & (kHeadDim - 1)));
    return l;
}
// Row m = b Sx + t (wave-uniform; host-checked: m H parts < 2^31) of a head-prep tile; outp is this
// lane's head output at row (b, t) = (0, 0), rsp its rstd at row 0.
__device__ inline void head_prep_store(const DmaParams& p, const HeadPrepLane& l, int m, int b, int t, int64_t nq,
                                       float4 y, const float* tab_row, bf16* outp, float* rsp) {
    const int d0 = (int)(nq & (kHeadDim - 1));
    if (l.gamma) {
        float4 cs = make_float4(0.f, 0.f, 0.f, 0.f), sn = cs;
        if (l.rope) rope_tab4(d0, p.hp.rope_dims, tab_row, cs, sn);
        const float r = head_norm_rope4(y, l.g, l.rope, d0, p.hp.rope_dims, p.hp.eps, cs, sn);
        if (d0 == 0) rsp[m * p.hp.H * p.hp.parts] = r;
    }
    const bf16 o[4] = {(bf16)y.x, (bf16)y.y, (bf16)y.z, (bf16)y.w};
    *reinterpret_cast<uint2*>(outp + ((int64_t)b * p.hp.H * p.hp.Sx + t) * kHeadDim) = __builtin_bit_cast(uint2, o);
}

// The attention dO epilogue at row m (main rows), output column nq (a multiple of 4 below N) with
// final values v: the bf16 head-major copy and, summed over the head's aligned 16-lane group (every
// lane of which takes this path: rows and 64-column heads are uniform over it), the row dots.
__device__ inline void attn_dot_store(const DmaParams& p, int64_t m, int64_t nq, const float4& v) {
    const unsigned sq = (unsigned)p.ad.Sq, b = (unsigned)m / sq, t = (unsigned)m - b * sq;
    const int d0 = (int)(nq & (kHeadDim - 1));
    const int64_t row = ((int64_t)b * p.ad.H + (nq >> 6)) * sq + t;   // kHeadDim = 64
    const int64_t idx = row * kHeadDim + d0;
    const uint2 a1 = *reinterpret_cast<const uint2*>(p.ad.o1 + idx);
    const uint2 a2 = *reinterpret_cast<const uint2*>(p.ad.o2 + idx);
    const bf16 o[4] = {(bf16)v.x, (bf16)v.y, (bf16)v.z, (bf16)v.w};
    *reinterpret_cast<uint2*>(p.ad.doh + idx) = __builtin_bit_cast(uint2, o);
    const float s1 = group16_sum(dot4_bf16(v, a1)), s2 = group16_sum(dot4_bf16(v, a2));
    if (d0 == 0) {
        p.ad.dn1[row] = s1;
        p.ad.dn2[row] = s2;
    }
}

// The SwiGLU backward epilogue at row m (main rows), output column nq (a multiple of 4 below N = I)
// with final values v = dG: both halves of the up-projection's dU from the bf16 [val | glu] row.
__device__ inline void swiglu_bwd_store(const DmaParams& p, int64_t m, int64_t nq, const float4& v) {
    const int64_t o = m * 2 * p.sb.I + nq;
    const float4 val = bf16x4_to_f4(*reinterpret_cast<const uint2*>(p.sb.F + o));
    const float4 glu = bf16x4_to_f4(*reinterpret_cast<const uint2*>(p.sb.F + o + p.sb.I));
    float4 dv, dgl;
    swiglu_bwd4(val, glu, v, dv, dgl);
    store_du4(p.sb.du + o, dv, p.sb.dsc, nq);
    store_du4(p.sb.du + o + p.sb.I, dgl, p.sb.dsc, p.sb.I + nq);
}

// The store phase of one staged-epilogue pass over tile rows [rb, rb + ER) (staged in st, EROW
// floats per row): thread tid stores chunk column cq (output column nq, column factors kq) of tile
// rows tid / CPR + i NT / CPR. With 256-column tiles a wave holds one row, which the paired SwiGLU
// and the head preparation rely on.
template <int BN, int NT, int ER, int EROW, bool HP, bool XE = false>
__device__ inline void staged_store(const DmaParams& p, const float* st, int64_t m0, int64_t n0, int rb, int64_t Mt,
                                    int z, int tid, int cq, int64_t nq, const EpiCols& kq, bool sw_tile, bool hp_tile,
                                    const HeadPrepLane& hl, const float* tabs) {
    constexpr int CPR = BN / 4, RS = NT / CPR, IT = ER * CPR / NT;
    static_assert(NT % CPR == 0 && (ER * CPR) % NT == 0, "a thread's chunk column must not change between rows");
    // the thread's first row: with one row per wave, a wave-uniform value
    const int r0 = CPR == 64 ? __builtin_amdgcn_readfirstlane(tid / CPR) : tid / CPR;
    const int64_t mf = m0 + rb + r0;
    const bool main_col = nq < p.N;
    const EpiRow er = epi_row(p, main_col && mf < p.M ? mf : 0, main_col ? nq : 0);
    const bool lo = cq < 128;
    bf16* gp = nullptr;
    if (BN == 256 && sw_tile) gp = p.sw_g + mf * p.sw_ldg + (lo ? nq : nq - p.sw_half + 2);
    [[maybe_unused]] int hb = 0, ht = 0;
    [[maybe_unused]] bf16* outp = nullptr;
    [[maybe_unused]] float* rsp = nullptr;
    if constexpr (HP) {
        if (hp_tile) {
            hb = (int)mf / p.hp.Sx;
            ht = (int)mf - hb * p.hp.Sx;
            const int h = (int)(nq - (int64_t)hl.k * p.hp.dim) >> 6;   // kHeadDim = 64
            outp = hl.out + (int64_t)h * p.hp.Sx * kHeadDim + (nq & (kHeadDim - 1));
            rsp = p.hp.rstd + (int64_t)h * p.hp.parts + hl.k;
        }
    }
    for (int it = 0; it < IT; ++it) {
        const int r = r0 + it * RS, dr = it * RS;
        const int64_t m = mf + dr;
        if constexpr (HP) {
            if (it) {
                ht += RS;
                while (ht >= p.hp.Sx) { ht -= p.hp.Sx; ++hb; }
            }
        }
        if (m >= Mt || nq >= p.Nt) continue;
        const float4 a = *reinterpret_cast<const float4*>(st + r * EROW + cq);
        if (p.ws) {
            *reinterpret_cast<float4*>(p.ws + (int64_t)z * Mt * p.Nt + m * p.Nt + nq) = a;
            continue;
        }
        const bool main_row = m < p.M;
        const float4 v = main_row && main_col ? epilogue_main4(p, er, dr, a, kq) : epilogue_vec4(p, m, nq, a, kq);
        if (BN == 256 && sw_tile && main_row) swiglu_pair_store(p, gp + (int64_t)dr * p.sw_ldg, lo, v);
        if constexpr (HP)
            if (hp_tile && main_row) head_prep_store(p, hl, (int)m, hb, ht, nq, v, tabs + (rb + r) * p.hp.rope_dims, outp, rsp);
        if constexpr (XE) {   // the backward epilogues: their own instantiations (register use)
            if (p.ad.doh && main_row && main_col) attn_dot_store(p, m, nq, v);
            if (p.sb.du && main_row && main_col) swiglu_bwd_store(p, m, nq, v);
        }
    }
}

// HP: the per-head q/k preparation instantiation (128 x 256 bf16 tiles): the staged epilogue takes
// the tile in two passes of 64 rows and keeps the tile rows' RoPE table rows in LDS past them.
// XE: the instantiation that also runs the backward epilogues (DmaParams::ad / sb); the others do
// not carry their code, which costs registers.
template <int BM, int BN, int WMW, int STAGES, bool BF16, int NW = 4, bool KN = false, int BQ = 0, bool HP = false,
          bool XE = false>
__global__ __launch_bounds__(NW * 64) void gemm_dma_kernel(DmaParams p) {
    constexpr int NT = NW * 64;
    constexpr int WNW = NW / WMW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    // MFMA block: bf16 uses v_mfma_f32_32x32x16_bf16 (twice the sustained rate of the 16x16x32
    // form on gfx950), f32 uses v_mfma_f32_16x16x4_f32
    constexpr int MT = BF16 ? 32 : 16;
    constexpr int FM = WTM / MT, FN = WTN / MT;
    constexpr int AE = BF16 ? 16 : 4;   // accumulator registers per block and lane
    constexpr int NA = BM * 8 / NT, NB = BN * 8 / NT;                // 16-byte chunks per thread per tile
    constexpr int LPT = NA + NB;                                     // DMA instructions per thread per tile
    constexpr int CE = BF16 ? 8 : 4;                                 // elements per chunk
    constexpr int EB = BF16 ? 2 : 4;                                 // bytes per element
    constexpr int BKE = 8 * CE;                                      // K elements per tile
    constexpr int STAGE_BYTES = (BM + BN) * kRow;
    // epilogue staging: the accumulators pass through LDS in row blocks of ER rows (a multiple of
    // the wave tile height), rows padded by 8 floats so the two row groups a store instruction
    // writes fall into different banks
    constexpr int EROW = BN + 8;
    constexpr int ER_FIT = (STAGES * STAGE_BYTES) / (EROW * 4);
    constexpr int ER = HP ? WTM : (ER_FIT >= BM ? BM : (ER_FIT / WTM) * WTM);
    static_assert(ER >= WTM, "epilogue staging does not fit");
    static_assert(!HP || (BF16 && BN == 256 && !KN && BQ == 0 && NT % 64 == 0 &&
                          (ER * EROW + BM * kHeadDim) * 4 <= STAGES * STAGE_BYTES),
                  "head preparation needs bf16 256-column tiles and room for the RoPE rows");
    static_assert(NA >= 1 && NB >= 1 && FM >= 1 && FN >= 1, "tile too small");
    static_assert(STAGES >= 2 && STAGES <= 4 && (STAGES - 1) * LPT < 64, "pipeline depth");
    static_assert(!KN || (BF16 && BN % 64 == 0), "a [K][N] B operand needs bf16 and whole 64-column sub-tiles");
    static_assert(BQ == 0 || (BF16 && !KN), "decoded B operands are bf16-compute, [N][K] only");
    constexpr int NBQ = BQ == 2 ? BN * 4 / NT : 0;             // Q8_0 quant chunks per thread per tile
    static_assert(BQ != 2 || (NBQ >= 1 && NB - NBQ - 1 >= 0 && NW * 64 >= BN &&
                              BN * 64 + NW * 256 + (NB - NBQ - 1) * NT * 16 <= BN * kRow),
                  "Q8_0 tile layout does not fit the bf16 B region");
    // The stages are consecutive STAGE_BYTES regions of one LDS array, each always addressed at a
    // compile-time offset. Every LDS write of the K loop is an inline-asm DMA, so the compiler
    // inserts no waits of its own; the loop orders DMA and reads with vmcnt waits and barriers.
    __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE_BYTES];

    const int64_t Mt = p.M + p.Mx;
    const int tiles_m = (int)((Mt + BM - 1) / BM), tiles_n = (int)((p.Nt + BN - 1) / BN);
    // This workgroup's item (split z, tile bid). Dispatch deals workgroups out to the 8 XCDs
    // round-robin in linear order (x fastest), so XCD c runs the linear ids L with L % 8 == c; it
    // takes the contiguous run [c T/8, (c+1) T/8) of the T items in (split, raster) order, so the
    // tiles of one split's K range that share A rows and B panels run on one XCD and share its L2.
    const int nwg = gridDim.x;   // tiles rounded up to a multiple of 8
    const int L = blockIdx.x + nwg * blockIdx.y;
    const int item = (L & 7) * ((nwg * (int)gridDim.y) >> 3) + (L >> 3);
    const int z = __builtin_amdgcn_readfirstlane(item / nwg);   // uniform: scalar operands derive from it
    const int bid = __builtin_amdgcn_readfirstlane(item - z * nwg);
    if (bid >= tiles_m * tiles_n) return;
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in_g = bid - group * per_group;
    const int tm = first_m + in_g % gsz, tn = in_g / gsz;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave % WMW) * WTM, wn0 = (wave / WMW) * WTN;

    const int KT = (int)(p.K / BKE);
    const int kt0 = z * p.kps;
    const int Tm = max(0, min(KT, kt0 + p.kps) - kt0);
    const bool ext = p.K2 > 0 && z == (int)gridDim.y - 1;
    const int T = Tm + (ext ? 1 : 0);
    const int64_t k0 = (int64_t)kt0 * BKE;

    // LDS destination (M0) of DMA q of this wave in stage 0; stage s adds s * STAGE_BYTES
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
    uint32_t dst[LPT];
#pragma unroll
    for (int q = 0; q < NA; ++q) dst[q] = lds_base + (q * NT + wave * 64) * 16;
#pragma unroll
    for (int q = 0; q < NB; ++q) dst[NA + q] = lds_base + BM * kRow + (q * NT + wave * 64) * 16;

    // Source of the chunk this thread DMAs into slot (q*NT + tid) of the A / B region of a stage:
    // row = slot/8, logical chunk kc = (slot%8) ^ swz(row).
    const char* ag[NA];    // main-segment chunk pointer at the split's first tile
    const char* a2g[NA];   // second-segment chunk pointer (zero page when past K2)
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gm = m0 + row;
        if (gm >= Mt) gm = 0;   // clamped: this output row is never stored
        if (gm < p.M) {
            ag[q] = static_cast<const char*>(p.A) + (gm * p.lda + k0 + kc * CE) * EB;
            a2g[q] = (kc * CE < p.K2) ? static_cast<const char*>(p.A2) + (gm * p.lda2 + kc * CE) * EB
                                      : static_cast<const char*>(p.zero);
        } else {
            const int64_t xr = gm - p.M;
            ag[q] = static_cast<const char*>(p.Ax) + (xr * p.ldax + k0 + kc * CE) * EB;
            a2g[q] = (kc * CE < p.K2) ? static_cast<const char*>(p.A2x) + (xr * p.lda2x + kc * CE) * EB
                                      : static_cast<const char*>(p.zero);
        }
    }
    const char* bg[NB];
    const char* b2g[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gn = tile_col_bn<BN>(p, n0, row);
        if (gn >= p.Nt) gn = 0;
        bg[q] = gn < p.N ? static_cast<const char*>(p.B) + (gn * p.ldb + k0 + kc * CE) * EB
                         : static_cast<const char*>(p.Bx) + ((gn - p.N) * p.ldbx + k0 + kc * CE) * EB;
        b2g[q] = (kc * CE < p.K2 && gn < p.N) ? static_cast<const char*>(p.B2) + (gn * p.ldb2 + kc * CE) * EB
                                              : static_cast<const char*>(p.zero);
    }

    // Main-segment loads through buffer descriptors when the operand extents allow it and the
    // tile's rows come from one source (A only, or the extra rows Ax only); otherwise, and for the
    // second segment, per-lane global addresses.
    const bool use_buf = p.a_bytes != 0 && p.b_bytes != 0 && (p.Nx == 0 || p.bx_bytes != 0);
    const int a_src = !use_buf ? 0 : (p.Mx == 0 || m0 + BM <= p.M) ? 1 : (m0 >= p.M && m0 + BM <= Mt && p.ax_bytes) ? 2 : 0;
    const u32x4 rs_a = buffer_rsrc(a_src == 2 ? p.Ax : p.A, a_src == 2 ? p.ax_bytes : p.a_bytes);
    const u32x4 rs_b = buffer_rsrc(p.B, p.b_bytes), rs_bx = buffer_rsrc(p.Bx, p.bx_bytes);
    uint32_t aoff[NA], boff[NB];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gm = m0 + row;
        if (gm >= Mt) gm = 0;
        aoff[q] = a_src == 2 ? (uint32_t)(((gm - p.M) * p.ldax + kc * CE) * EB) : (uint32_t)((gm * p.lda + kc * CE) * EB);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gn = tile_col_bn<BN>(p, n0, row);
        if (gn >= p.Nt) gn = 0;
        boff[q] = gn < p.N ? (uint32_t)((gn * p.ldb + kc * CE) * EB) : (uint32_t)(((gn - p.N) * p.ldbx + kc * CE) * EB);
    }
    // the 8 rows of B slot (q, wave) start at n0 + (q * NT + 64 wave) / 8: one source per slot
    // (N % 8 == 0), chosen on the scalar unit
    unsigned bx_mask = 0;   // bit q: slot q's rows are extra columns (fixed over the K loop)
    if constexpr (KN) {
        // [K][N] B: slot s of the B region is sub-tile s / 512, row k = (s % 512) / 8 of the K tile,
        // logical chunk (s % 8) ^ swz(k): 8 columns at n0 + 64 (s / 512) + 8 chunk (columns past N
        // read a valid column; their results are never stored). The K tile moves in soff. A wave's
        // slot q lies in one sub-tile; with extra columns (N % 64 == 0) a sub-tile at or past N reads
        // them from Bx, [K][Nx] with row pitch ldbx.
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int s = q * NT + tid, t = s >> 9, k = (s & 511) >> 3, kc = (s & 7) ^ swz(k);
            const bool extra = p.Nx > 0 && n0 + 64 * ((q * NT + wave * 64) >> 9) >= p.N;   // wave-uniform
            int64_t gn = n0 + 64 * t + 8 * kc;
            if (extra) {
                bx_mask |= 1u << q;
                int64_t gx = gn - p.N;
                if (gx + 8 > p.Nx) gx = p.Nx - 8;
                boff[q] = (uint32_t)(((int64_t)k * p.ldbx + gx) * 2);
            } else {
                if (gn + 8 > p.N) gn = p.N - 8;
                boff[q] = (uint32_t)(((int64_t)k * p.ldb + gn) * 2);
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int64_t r0 = tile_col_bn<BN>(p, n0, (q * NT + wave * 64) / 8);
            if (r0 < p.Nt && r0 >= p.N) bx_mask |= 1u << q;
        }
    }
    auto slot_bx = [&](int q) { return ((bx_mask >> q) & 1u) != 0; };
    // Q8_0: quant slot s = q NT + tid holds row s / 4, physical chunk s % 4 = logical chunk
    // kc ^ qswz(row) (16 quant bytes); lane l of wave w loads row 64 w + l's two block scales
    uint32_t qoff[BQ == 2 ? NBQ : 1] = {};
    uint32_t soff_sc = 0;
    u32x4 rs_bs = {};
    if constexpr (BQ == 2) {
#pragma unroll
        for (int q = 0; q < NBQ; ++q) {
            const int s = q * NT + tid, row = s >> 2, kc = (s & 3) ^ qswz(row);
            int64_t gn = n0 + row;
            if (gn >= p.N) gn = 0;   // clamped: this output column is never stored
            qoff[q] = (uint32_t)(gn * p.ldb + kc * 16);
        }
        const int srow = wave * 64 + lane;
        const int64_t gn = n0 + srow;
        soff_sc = srow < BN && gn < p.N ? (uint32_t)(gn * p.ldbs * 2) : 0xFFFFFFF0u;
        rs_bs = buffer_rsrc(p.Bs, p.bs_bytes);
    }

    auto issue = [&](auto s_c, int t) {
        constexpr uint32_t so_lds = (uint32_t)((decltype(s_c)::value % STAGES) * STAGE_BYTES);
        if (t < Tm) {
            const uint32_t so = (uint32_t)((k0 + (int64_t)t * BKE) * EB);
            if (a_src != 0) {
#pragma unroll
                for (int q = 0; q < NA; ++q) dma16b(rs_a, aoff[q], so, dst[q] + so_lds);
            } else {
#pragma unroll
                for (int q = 0; q < NA; ++q) dma16(ag[q] + (int64_t)t * (BKE * EB), dst[q] + so_lds);
            }
            if constexpr (BQ == 2) {   // quants, block scales, then the padding loads
                const uint32_t kq = (uint32_t)(k0 + (int64_t)t * BKE);   // bytes into the quant rows
#pragma unroll
                for (int q = 0; q < NBQ; ++q) dma16b(rs_b, qoff[q], kq, dst[NA + q] + so_lds);
                const uint32_t sc0 = lds_base + BM * kRow + BN * 64 + so_lds;
                dma4b(rs_bs, soff_sc, kq / 16, sc0 + (uint32_t)wave * 256u);
#pragma unroll
                for (int q = 0; q < NB - NBQ - 1; ++q)
                    dma16b(rs_bs, 0xFFFFFFF0u, 0u, sc0 + NW * 256 + (uint32_t)((q * NT + wave * 64) * 16));
            } else if constexpr (KN) {   // always through the descriptor: the K tile is a row offset
                const uint32_t sob = (uint32_t)((k0 + (int64_t)t * BKE) * p.ldb * 2);
                const uint32_t sobx = (uint32_t)((k0 + (int64_t)t * BKE) * p.ldbx * 2);
#pragma unroll
                for (int q = 0; q < NB; ++q)
                    dma16b(pick_rsrc(slot_bx(q), rs_bx, rs_b), boff[q], slot_bx(q) ? sobx : sob, dst[NA + q] + so_lds);
            } else if (a_src != 0) {
#pragma unroll
                for (int q = 0; q < NB; ++q) dma16b(pick_rsrc(slot_bx(q), rs_bx, rs_b), boff[q], so, dst[NA + q] + so_lds);
            } else {
#pragma unroll
                for (int q = 0; q < NB; ++q) dma16(bg[q] + (int64_t)t * (BKE * EB), dst[NA + q] + so_lds);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) dma16(a2g[q], dst[q] + so_lds);
#pragma unroll
            for (int q = 0; q < NB; ++q) dma16(b2g[q], dst[NA + q] + so_lds);
        }
    };

    typedef float accv __attribute__((__vector_size__(AE * sizeof(float))));
    accv acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < AE; ++v) acc[i][j][v] = 0.f;

    // operand fragments: lane l reads 16 bytes, chunk kc of row (l % MT) of a block
    auto frag = [&](const char* base, int row, int kc) {
        return base + row * kRow + ((kc ^ swz(row)) << 4);
    };
    // B fragment of lane (row n, K step ks, half g) decoded to bf16 from f16 (BQ 1) or Q8_0 (BQ 2):
    // the same RNE of the exact decoded value as the weight's bf16 working copy
    auto dq_frag = [&](const char* Bs, int n, int ks, int g, int kc) __attribute__((always_inline)) -> bf16x8 {
        bf16x8 o;
        if constexpr (BQ == 1) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
            const h8 h = *reinterpret_cast<const h8*>(frag(Bs, n, kc));
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (__bf16)(float)h[e];
        } else if constexpr (BQ == 2) {
            const uint2 qv = *reinterpret_cast<const uint2*>(Bs + n * 64 + ((ks ^ qswz(n)) << 4) + 8 * g);
            const float sc = (float)*reinterpret_cast<const _Float16*>(Bs + BN * 64 + n * 4 + (ks >> 1) * 2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const unsigned w = e < 4 ? qv.x : qv.y;
                const int q = (int)(signed char)(w >> (8 * (e & 3)));
                o[e] = (__bf16)(sc * (float)q);
            }
        }
        return o;
    };
    auto compute = [&](const char* As, bool deq) __attribute__((always_inline)) {
        const char* Bs = As + BM * kRow;
        if constexpr (BF16) {
            // 32x32x16: lane l holds row l%32, k = 8*(l/32) + e; four K steps of 16 per tile
            // all fragments of the tile are read first (distinct registers), so the MFMAs of each
            // K step wait only for their own operands while later reads are still in flight
            const int r = lane & 31, g = lane >> 5;
            bf16x8 af[4][FM], bfr[4][FN];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int kc = 2 * ks + g;
#pragma unroll
                for (int i = 0; i < FM; ++i) af[ks][i] = *reinterpret_cast<const bf16x8*>(frag(As, wm0 + 32 * i + r, kc));
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    if constexpr (KN) {
                        // lane: column nb + lane%32, K rows 16 ks + 8 (lane/32) .. +7 of the sub-tile
                        const int nb = wn0 + 32 * j;
                        const char* sub = Bs + (nb >> 6) * (64 * kRow);
                        const int nl = (nb & 63) + 16 * ((lane >> 4) & 1), kb = 16 * ks + 8 * g;
                        bfr[ks][j] = cat44(ld_tr(sub, kb, nl, lane), ld_tr(sub, kb + 4, nl, lane));
                    } else if (BQ != 0 && deq) {
                        bfr[ks][j] = dq_frag(Bs, wn0 + 32 * j + r, ks, g, kc);
                    } else {
                        bfr[ks][j] = *reinterpret_cast<const bf16x8*>(frag(Bs, wn0 + 32 * j + r, kc));
                    }
                }
            }
            // keep the reads ahead of the MFMAs (the LDS counter tracks at most 15 reads, so the
            // first half's MFMAs can start with the second half's reads still outstanding)
            __builtin_amdgcn_sched_barrier(0);
            if (p.prio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], bfr[ks][j], acc[i][j], 0, 0, 0);
                if (ks == 1) __builtin_amdgcn_sched_barrier(0);
            }
            if (p.prio) __builtin_amdgcn_s_setprio(0);
        } else {
            // 16x16x4 f32: lane l holds row l%16; a 16-byte chunk feeds four K steps
            const int r = lane & 15, g = lane >> 4;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int kc = 4 * s + g;
                f32x4 af[FM], bfr[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const f32x4*>(frag(As, wm0 + 16 * i + r, kc));
#pragma unroll
                for (int j = 0; j < FN; ++j) bfr[j] = *reinterpret_cast<const f32x4*>(frag(Bs, wn0 + 16 * j + r, kc));
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int j = 0; j < FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], bfr[j][e], acc[i][j], 0, 0, 0);
            }
        }
    };
    // output row (within a block) of accumulator register v of this lane; the column is lane % MT
    auto out_row = [&](int v) { return BF16 ? 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3) : 4 * (lane >> 4) + v; };
    // prescale: the main segment's sums times colscale[n], before the second segment is added
    auto scale_acc = [&] {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn0 + MT * j + (lane & (MT - 1));
            const float c = n < p.N ? p.colscale[n] : 0.f;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int v = 0; v < AE; ++v) acc[i][j][v] = acc[i][j][v] * c;
        }
    };

    // prologue: STAGES-1 tiles in flight; tile t always lives in stage t % STAGES
    static_for<STAGES - 1>([&](auto s) {
        if (decltype(s)::value < T) issue(s, decltype(s)::value);
    });
    for (int t0 = 0; t0 < T; t0 += STAGES) {
        static_for<STAGES>([&](auto s) {
            const int t = t0 + decltype(s)::value;
            if (t >= T) return;
            // tile t has landed once at most min(STAGES-2, T-1-t) later tiles are outstanding
            const int later = min(STAGES - 2, T - 1 - t);
            if (later >= STAGES - 2) wait_vmcnt<(STAGES - 2) * LPT>();
            else if constexpr (STAGES >= 3) {
                if (later == 1) wait_vmcnt<LPT>();
                else wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();
            }
            // tile t visible to all waves; every wave is done with tile t-1. A bare s_barrier: the
            // fence __syncthreads adds would wait for every in-flight DMA (vmcnt 0), not just tile t.
            __asm__ volatile("s_barrier" ::: "memory");
            if (t + STAGES - 1 < T) issue(IC<decltype(s)::value + STAGES - 1>{}, t + STAGES - 1);
            if (p.prescale && t == Tm) scale_acc();
            compute(lds + decltype(s)::value * STAGE_BYTES, t < Tm);
        });
    }
    if (p.prescale && !ext) scale_acc();   // a split without the second segment

    if (p.ws && p.counters) {  // split-K with in-kernel reduction: coherent partials, element-wise
        float* w = p.ws + (int64_t)z * Mt * p.Nt;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn0 + MT * j + (lane & (MT - 1));
            if (n >= p.Nt) continue;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int v = 0; v < AE; ++v) {
                    const int64_t m = m0 + wm0 + MT * i + out_row(v);
                    if (m < Mt) st_coherent(w + m * p.Nt + n, acc[i][j][v]);
                }
        }
        // The last split of this tile to arrive sums the partials in split order (deterministic:
        // independent of the arrival order) and runs the epilogue; nobody waits for anybody.
        __shared__ int s_last;
        if (!arrive_last(&p.counters[bid], (int)gridDim.y, &s_last)) return;
        const int splits = (int)gridDim.y;
        for (int e = tid; e < BM * BN; e += NT) {
            const int64_t m = m0 + e / BN, n = n0 + e % BN;
            if (m >= Mt || n >= p.Nt) continue;
            float sum = 0.f;
            for (int zz = 0; zz < splits; ++zz) sum += ld_coherent(p.ws + (int64_t)zz * Mt * p.Nt + m * p.Nt + n);
            epilogue_elem(p, m, n, sum);
        }
        return;
    }

    if (!p.vec_epi) {   // element-wise epilogue (unaligned outputs)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn0 + MT * j + (lane & (MT - 1));
            if (n >= p.Nt) continue;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int v = 0; v < AE; ++v) {
                    const int64_t m = m0 + wm0 + MT * i + out_row(v);
                    if (m >= Mt) continue;
                    if (p.ws) p.ws[(int64_t)z * Mt * p.Nt + m * p.Nt + n] = acc[i][j][v];
                    else epilogue_elem(p, m, n, acc[i][j][v]);
                }
        }
        return;
    }

    // Staged epilogue: the waves owning rows [rb, rb + ER) of the tile write their accumulators to
    // LDS (row-major, padded rows), then every thread stores 16-byte row chunks: whole cache lines
    // per wave instead of one scattered element per lane and register. A thread's chunk column cq
    // is the same in every row (NT is a multiple of the chunks per row), so its column factors are
    // loaded once, ahead of the output stores. A paired SwiGLU tile's val-column threads also read
    // the matching glu chunk 128 columns on and write g.
    constexpr int CPR = BN / 4;   // 16-byte chunks per row
    static_assert(NT % CPR == 0, "a thread's chunk column must not change between rows");
    const int cq = (tid % CPR) * 4;
    const int64_t nq = tile_col_bn<BN>(p, n0, cq);
    const EpiCols kq = epi_cols(p, nq);
    const bool sw_tile = BN == 256 && p.sw_half > 0 && n0 < 2 * p.sw_half;   // workgroup-uniform
    epi_cols_ready(kq);
    float* st = reinterpret_cast<float*>(lds);
    __syncthreads();   // every wave is done reading the last K tile
    // head preparation (workgroup-uniform: every main-column tile lies inside one part): this
    // lane's gains, and the tile rows' RoPE table rows staged past the accumulator rows, loaded
    // ahead of the output stores
    const bool hp_tile = HP && n0 < p.N;
    HeadPrepLane hl{};
    float* tabs = st + ER * EROW;
    if constexpr (HP) {
        if (hp_tile) {
            hl = head_prep_lane(p, n0, nq);
            if (hl.rope) {
                const int R4 = p.hp.rope_dims / 4;
                for (int i = tid; i < BM * R4; i += NT) {
                    const int r = i / R4, c = i - r * R4;
                    const int64_t m = min(m0 + r, p.M - 1);
                    const unsigned t = (unsigned)m % (unsigned)p.hp.Sx;
                    *reinterpret_cast<float4*>(tabs + r * p.hp.rope_dims + 4 * c) =
                        *reinterpret_cast<const float4*>(p.hp.tab + t * p.hp.rope_dims + 4 * c);
                }
            }
            asm volatile("" ::"v"(hl.g.x), "v"(hl.g.y), "v"(hl.g.z), "v"(hl.g.w));   // loaded before the stores
        }
    }
#pragma unroll
    for (int rb = 0; rb < BM; rb += ER) {
        if (wm0 >= rb && wm0 < rb + ER) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int c = wn0 + MT * j + (lane & (MT - 1));
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int v = 0; v < AE; ++v) st[(wm0 - rb + MT * i + out_row(v)) * EROW + c] = acc[i][j][v];
            }
        }
        __syncthreads();
        staged_store<BN, NT, ER, EROW, HP, XE>(p, st, m0, n0, rb, Mt, z, tid, cq, nq, kq, sw_tile, hp_tile, hl, tabs);
        if (rb + ER < BM) __syncthreads();
    }
}

// 256 x 256 tiles for bf16 operands, one workgroup of 8 waves per CU (128 KiB of LDS in two
// stages). Per K tile of 64 a CU then moves 64 KiB from L2 for 8.4 MFLOP, half the bytes per flop
// of two 128 x 128 workgroups (which need the CU's whole 64 B/clk vector-memory path at the MFMA
// peak), and its waves own 64 x 128 blocks (2 x 4 MFMA blocks of 32 x 32), which cut LDS reads per
// flop by a quarter against 64 x 64.
//
// Every operand load goes through a buffer descriptor with a 32-bit per-lane offset (no 64-bit
// pointers, which would not leave room for the 128 accumulator registers): host-checked extents
// below 4 GiB. A (q, wave) DMA slot covers 8 consecutive rows, so with M % 8 == 0 its rows all come
// from A or all from the extra rows Ax, a choice made per slot on the scalar unit. Rows past the
// end are clamped to the last valid row of the same source. The rank segment (K2 <= 64) has its
// own descriptors; its chunks past K2 get an offset beyond the descriptor extent, which loads zeros.
struct BigSeg {
    uint32_t off[4];
};

template <bool KN, int NW = 8, bool XE = false>   // XE: as for gemm_dma_kernel
__global__ __launch_bounds__(NW * 64) void gemm_big_kernel(DmaParams p) {
    constexpr int BM = 256, BN = 256, NT = NW * 64, WMW = 4;
    constexpr int WTM = BM / WMW, WTN = BN / (NW / WMW);   // 64 x 128 (8 waves), 64 x 64 (16)
    constexpr int FM = WTM / 32, FN = WTN / 32;             // MFMA blocks per wave
    constexpr int NA = BM * 8 / NT, NB = BN * 8 / NT;       // DMA chunks per thread and tile
    constexpr int RPQ = NT / 8;                             // tile rows per DMA slot q
    constexpr int LPT = NA + NB;
    constexpr int STAGES = 2;
    constexpr int STAGE_BYTES = (BM + BN) * kRow;           // 64 KiB
    constexpr int EROW = BN + 8;
    constexpr int ER = 64;                                  // epilogue rows staged per pass
    static_assert(ER * EROW * 4 <= STAGES * STAGE_BYTES, "epilogue staging does not fit");
    __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE_BYTES];

    const int64_t Mt = p.M + p.Mx;
    const int tiles_m = (int)((Mt + BM - 1) / BM), tiles_n = (int)((p.Nt + BN - 1) / BN);
    // This workgroup's item (split z, tile bid). Dispatch deals workgroups out to the 8 XCDs
    // round-robin in linear order (x fastest), so XCD c runs the linear ids L with L % 8 == c; it
    // takes the contiguous run [c T/8, (c+1) T/8) of the T items in (split, raster) order, so the
    // tiles of one split's K range that share A rows and B panels run on one XCD and share its L2.
    const int nwg = gridDim.x;   // tiles rounded up to a multiple of 8
    const int L = blockIdx.x + nwg * blockIdx.y;
    const int item = (L & 7) * ((nwg * (int)gridDim.y) >> 3) + (L >> 3);
    const int z = __builtin_amdgcn_readfirstlane(item / nwg);   // uniform: scalar operands derive from it
    const int bid = __builtin_amdgcn_readfirstlane(item - z * nwg);
    if (bid >= tiles_m * tiles_n) return;
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in_g = bid - group * per_group;
    const int tm = first_m + in_g % gsz, tn = in_g / gsz;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave % WMW) * WTM, wn0 = (wave / WMW) * WTN;

    const int KT = (int)(p.K / 64);
    const int kt0 = z * p.kps;
    const int Tm = max(0, min(KT, kt0 + p.kps) - kt0);
    const bool ext = p.K2 > 0 && z == (int)gridDim.y - 1;
    const int T = Tm + (ext ? 1 : 0);
    const uint32_t k0b = (uint32_t)kt0 * 128u;   // byte offset of the split's first K tile

    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
    const u32x4 rs_a = buffer_rsrc(p.A, p.a_bytes), rs_ax = buffer_rsrc(p.Ax, p.ax_bytes);
    const u32x4 rs_b = buffer_rsrc(p.B, p.b_bytes), rs_bx = buffer_rsrc(p.Bx, p.bx_bytes);
    // the rank segment's descriptors: [rows][ld2] bf16, K2 valid columns
    const uint32_t a2_bytes = p.K2 > 0 ? (uint32_t)(((p.M - 1) * p.lda2 + p.K2) * 2) : 0u;
    const uint32_t a2x_bytes = p.K2 > 0 && p.Mx > 0 ? (uint32_t)(((p.Mx - 1) * p.lda2x + p.K2) * 2) : 0u;
    const uint32_t b2_bytes = p.K2 > 0 ? (uint32_t)(((p.N - 1) * p.ldb2 + p.K2) * 2) : 0u;
    const u32x4 rs_a2 = buffer_rsrc(p.A2, a2_bytes), rs_a2x = buffer_rsrc(p.A2x, a2x_bytes);
    const u32x4 rs_b2 = buffer_rsrc(p.B2, b2_bytes);
    constexpr uint32_t kNoData = 0xFFFFFFF0u;   // past every extent: loads zeros

    // per-thread DMA sources: slot s = q * NT + tid of the A (B) region, row s / 8, chunk kc. The 8
    // rows of slot (q, wave) start at m0 + (NT / 8) q + 8 wave, so their source is decided from
    // wave-uniform values (M % 8 == 0 when there are extra rows).
    BigSeg ao, a2o, bo, b2o;
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gm = m0 + row;
        if (gm >= Mt) gm = Mt - 1;
        const bool x = gm >= p.M;
        const int64_t lr = x ? gm - p.M : gm;
        ao.off[q] = (uint32_t)((lr * (x ? p.ldax : p.lda) + kc * 8) * 2);
        a2o.off[q] = kc * 8 < p.K2 ? (uint32_t)((lr * (x ? p.lda2x : p.lda2) + kc * 8) * 2) : kNoData;
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        const int s = q * NT + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gn = tile_col(p, n0, row);
        if (gn >= p.Nt) gn = p.Nt - 1;
        bo.off[q] = gn < p.N ? (uint32_t)((gn * p.ldb + kc * 8) * 2) : (uint32_t)(((gn - p.N) * p.ldbx + kc * 8) * 2);
        b2o.off[q] = kc * 8 < p.K2 && gn < p.N ? (uint32_t)((gn * p.ldb2 + kc * 8) * 2) : kNoData;
    }
    // wave-uniform, fixed over the K loop: bit q set when slot q's B rows are extra columns (N % 8
    // == 0), resp. its A rows extra rows (M % 8 == 0)
    unsigned bx_mask = 0, x_mask = 0;
#pragma unroll
    for (int q = 0; q < NB; ++q)
        if (min(tile_col(p, n0, RPQ * q + 8 * wave), p.Nt - 1) >= p.N) bx_mask |= 1u << q;
#pragma unroll
    for (int q = 0; q < NA; ++q)
        if (min(m0 + RPQ * q + 8 * wave, Mt - 1) >= p.M) x_mask |= 1u << q;
    auto slot_bx = [&](int q) { return ((bx_mask >> q) & 1u) != 0; };
    if constexpr (KN) {
        // [K][N] B: slot s of the B region is sub-tile s / 512 (64 columns), row k = (s % 512) / 8 of
        // the K tile, logical chunk (s % 8) ^ swz(k); columns past N read a valid column. A wave's
        // slot q lies in one sub-tile; with extra columns (N % 64 == 0) a sub-tile at or past N reads
        // them from Bx, [K][Nx] with row pitch ldbx.
        bx_mask = 0;
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int s = q * NT + tid, t = s >> 9, k = (s & 511) >> 3, kc = (s & 7) ^ swz(k);
            const bool extra = p.Nx > 0 && n0 + 64 * ((q * NT + wave * 64) >> 9) >= p.N;   // wave-uniform
            int64_t gn = n0 + 64 * t + 8 * kc;
            if (extra) {
                bx_mask |= 1u << q;
                int64_t gx = gn - p.N;
                if (gx + 8 > p.Nx) gx = p.Nx - 8;
                bo.off[q] = (uint32_t)(((int64_t)k * p.ldbx + gx) * 2);
            } else {
                if (gn + 8 > p.N) gn = p.N - 8;
                bo.off[q] = (uint32_t)(((int64_t)k * p.ldb + gn) * 2);
            }
        }
    }
    auto slot_x = [&](int q) { return ((x_mask >> q) & 1u) != 0; };

    auto issue = [&](auto s_c, int t) {
        constexpr uint32_t so_lds = (uint32_t)((decltype(s_c)::value % STAGES) * STAGE_BYTES);
        const uint32_t dst0 = lds_base + wave * 64 * 16 + so_lds;
        if (t < Tm) {
            const uint32_t so = k0b + (uint32_t)t * 128u;
#pragma unroll
            for (int q = 0; q < NA; ++q) dma16b(slot_x(q) ? rs_ax : rs_a, ao.off[q], so, dst0 + q * NT * 16);
            if constexpr (KN) {   // the K tile is a row offset of the [K][N] operand
                const uint32_t sob = (uint32_t)(((int64_t)kt0 + t) * 64 * p.ldb * 2);
                const uint32_t sobx = (uint32_t)(((int64_t)kt0 + t) * 64 * p.ldbx * 2);
#pragma unroll
                for (int q = 0; q < NB; ++q)
                    dma16b(pick_rsrc(slot_bx(q), rs_bx, rs_b), bo.off[q], slot_bx(q) ? sobx : sob,
                           dst0 + BM * kRow + q * NT * 16);
            } else {
#pragma unroll
                for (int q = 0; q < NB; ++q)
                    dma16b(pick_rsrc(slot_bx(q), rs_bx, rs_b), bo.off[q], so, dst0 + BM * kRow + q * NT * 16);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) dma16b(slot_x(q) ? rs_a2x : rs_a2, a2o.off[q], 0u, dst0 + q * NT * 16);
#pragma unroll
            for (int q = 0; q < NB; ++q) dma16b(rs_b2, b2o.off[q], 0u, dst0 + BM * kRow + q * NT * 16);
        }
    };

    typedef float accv __attribute__((__vector_size__(16 * sizeof(float))));
    accv acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    auto frag = [&](const char* base, int row, int kc) { return base + row * kRow + ((kc ^ swz(row)) << 4); };
    // two K steps of fragments at a time: the reads of steps 2-3 go out while steps 0-1 compute
    auto compute = [&](const char* As) {
        const char* Bs = As + BM * kRow;
        const int r = lane & 31, g = lane >> 5;
        bf16x8 af[2][FM], bfr[2][FN];
        auto load = [&](int ks, int slot) {
            const int kc = 2 * ks + g;
#pragma unroll
            for (int i = 0; i < FM; ++i) af[slot][i] = *reinterpret_cast<const bf16x8*>(frag(As, wm0 + 32 * i + r, kc));
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (KN) {
                    const int nb = wn0 + 32 * j;
                    const char* sub = Bs + (nb >> 6) * (64 * kRow);
                    const int nl = (nb & 63) + 16 * ((lane >> 4) & 1), kb = 16 * ks + 8 * g;
                    bfr[slot][j] = cat44(ld_tr(sub, kb, nl, lane), ld_tr(sub, kb + 4, nl, lane));
                } else {
                    bfr[slot][j] = *reinterpret_cast<const bf16x8*>(frag(Bs, wn0 + 32 * j + r, kc));
                }
            }
        };
        auto mma = [&](int slot) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
        };
        load(0, 0);
        load(1, 1);
        __builtin_amdgcn_sched_barrier(0);
        if (p.prio) __builtin_amdgcn_s_setprio(1);
        mma(0);
        load(2, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(1);
        load(3, 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(0);
        mma(1);
        if (p.prio) __builtin_amdgcn_s_setprio(0);
    };

    if (T > 0) issue(IC<0>{}, 0);
    for (int t0 = 0; t0 < T; t0 += STAGES) {
        static_for<STAGES>([&](auto s) {
            const int t = t0 + decltype(s)::value;
            if (t >= T) return;
            wait_vmcnt<0>();   // tile t landed (the only DMA group in flight)
            __asm__ volatile("s_barrier" ::: "memory");   // visible to all waves; tile t-1 consumed
            if (t + 1 < T) issue(IC<decltype(s)::value + 1>{}, t + 1);
            compute(lds + decltype(s)::value * STAGE_BYTES);
        });
    }

    // staged epilogue only (the host routes outputs that do not allow 16-byte stores elsewhere);
    // fixed chunk column per thread as in gemm_dma_kernel
    auto out_row = [&](int v) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); };
    constexpr int CPR = BN / 4;
    static_assert(NT % CPR == 0, "a thread's chunk column must not change between rows");
    const int cq = (tid % CPR) * 4;
    const int64_t nq = tile_col(p, n0, cq);
    const EpiCols kq = epi_cols(p, nq);
    const bool sw_tile = p.sw_half > 0 && n0 < 2 * p.sw_half;   // workgroup-uniform
    epi_cols_ready(kq);
    float* st = reinterpret_cast<float*>(lds);
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < BM; rb += ER) {
        if (wm0 == rb) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int c = wn0 + 32 * j + (lane & 31);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) st[(32 * i + out_row(v)) * EROW + c] = acc[i][j][v];
            }
        }
        __syncthreads();
        staged_store<BN, NT, ER, EROW, false, XE>(p, st, m0, n0, rb, Mt, z, tid, cq, nq, kq, sw_tile, false,
                                              HeadPrepLane{}, nullptr);
        if (rb + ER < BM) __syncthreads();
    }
}

// Sum of the split partials in split order, then the epilogue: 4 consecutive columns per thread
// when the outputs allow 16-byte accesses, one element otherwise.
__global__ __launch_bounds__(kThreads) void gemm_dma_splitk_reduce(DmaParams p, int splits) {
    const int64_t Mt = p.M + p.Mx;
    const int64_t plane = Mt * p.Nt;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    // the partials are loaded eight splits at a time (indices past the last split re-read it and
    // are not added), so a thread waits about splits / 8 memory round trips; the sums are added
    // in split order from zero either way
    if (p.vec_epi) {
        const int64_t e = idx * 4;
        if (e >= plane) return;
        float4 s = make_float4(0.f, 0.f, 0.f, 0.f);   // same sums as the element path
        for (int z = 0; z < splits; z += 8) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = *reinterpret_cast<const float4*>(p.ws + (int64_t)min(z + k, splits - 1) * plane + e);
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (z + k < splits) s = make_float4(s.x + v[k].x, s.y + v[k].y, s.z + v[k].z, s.w + v[k].w);
        }
        const int64_t m = e / p.Nt, n = e - m * p.Nt;
        epilogue_vec4(p, m, n, s);
        return;
    }
    if (idx >= plane) return;
    float s = 0.f;
    for (int z = 0; z < splits; z += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = p.ws[(int64_t)min(z + k, splits - 1) * plane + idx];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (z + k < splits) s += v[k];
    }
    const int64_t m = idx / p.Nt, n = idx - m * p.Nt;
    epilogue_elem(p, m, n, s);
}

// The split over K of a launch of `tiles` tiles with `slots` resident workgroups and KT K tiles,
// one rule for the launchers and for dma_rounds: split only when there are K tiles to spare (below
// 16, e.g. the 256-token context projection with K = 768, the split partials and their reduction
// launch cost more than the idle slots: 256 x 4608 x 768 measured 10.6 us unsplit, 16.9 us in 3
// splits), into at most 16 and at most slots / tiles parts, so splits x tiles <= slots; option
// gemm_splits forces a count. Returns the splits actually used (every split gets a whole share).
int split_count(const sa3k_ctx* ctx, int64_t tiles, int64_t slots, int KT, int* kps) {
    int splits = 1;
    if (ctx->gemm_split && tiles < slots && KT >= 16)
        splits = (int)std::min<int64_t>({(int64_t)16, KT / 4, std::max<int64_t>(1, slots / tiles)});
    if (ctx->gemm_splits > 0 && ctx->gemm_split) splits = std::min(ctx->gemm_splits, std::max(1, KT));
    const int per = std::max(1, (KT + splits - 1) / splits);
    if (kps) *kps = per;
    splits = std::max(1, (KT + per - 1) / per);
    // the bound the allocation-free entry point's scratch is sized by (kMaxSplitFloats)
    SA3K_REQUIRE(splits == 1 || ctx->gemm_splits > 0 || (int64_t)splits * tiles <= slots,
                 "GEMM split plan exceeds the resident slots");
    return splits;
}

// Whether a bf16 product of Mt x Nt x K takes the 256 x 256 tiles (one workgroup per CU): where
// they fill the chip about as evenly as 128 x 128 tiles (two per CU) do, or with option gemm_big 3
// for K >= 8192 (they need no split over K there, or fewer), always with gemm_big 2. Measured on
// MI355X at 2176 rows: FFN up-projection 2176 x 12288 x 1536 107 vs 111 us, 2176 x 6144 x 1536 52
// vs 56 us, 8192^3 877 vs 1057 us; the 2176 x 7680 QKV projection (270 tiles) 98 vs 62 us.
bool use_big_tiles(const sa3k_ctx* ctx, int64_t Mt, int64_t Nt, int64_t K) {
    if (ctx->gemm_big == 0 || Mt <= 32 || Nt <= 64) return false;
    const int64_t t256 = ceil_div(Mt, 256) * ceil_div(Nt, 256), t128 = ceil_div(Mt, 128) * ceil_div(Nt, 128);
    const double q256 = (double)t256 / (double)(ceil_div(t256, 256) * 256);
    const double q128 = (double)t128 / (double)(ceil_div(t128, 512) * 512);
    return ctx->gemm_big == 2 || (t256 >= 200 && q256 >= q128 - 0.02) || (ctx->gemm_big == 3 && K >= 8192);
}

// Keep the paired SwiGLU epilogue only where the launch computes each tile's final values in one
// workgroup and stores them through the staged epilogue: 256-column tiles, no split over K, a
// [N][K] bf16 B, N = 2 sw_half a multiple of 256 (every tile below N is paired), no extra rows and
// no accumulation into C. Otherwise sw_half is cleared and *sw_done left alone.
void settle_swiglu(DmaParams& p, int bn, int splits, bool kn, int bq) {
    if (p.sw_half <= 0) return;
    const bool ok = bn == 256 && splits == 1 && !kn && bq == 0 && p.vec_epi && !p.accumulate && p.Mx == 0 &&
                    p.N == 2 * p.sw_half && p.N % 256 == 0 && p.sw_g && p.sw_ldg % 4 == 0 &&
                    (uintptr_t)p.sw_g % 8 == 0;
    if (!ok) {
        p.sw_half = 0;
        return;
    }
    if (p.sw_done) *p.sw_done = 1;
    if (p.c_unfused_only) p.C = nullptr;
}

// Whether the per-head q/k preparation fits this launch: one workgroup per tile (no split over K),
// the staged epilogue, no extra rows, no accumulation, N = parts x dim with dim = H x 64 a multiple
// of 256 (so each 256-column tile lies in one part), M = B x Sx, RoPE dims a multiple of 8.
bool headprep_ok(const DmaParams& p, int splits) {
    const HeadPrep& h = p.hp;
    if (h.parts <= 0 || h.parts > 5 || splits != 1 || !p.vec_epi || p.accumulate || p.Mx != 0) return false;
    if (h.dim % 256 != 0 || h.H * kHeadDim != h.dim || p.N != (int64_t)h.parts * h.dim) return false;
    if (h.Sx <= 0 || p.M % h.Sx != 0 || p.M * h.H * h.parts >= ((int64_t)1 << 31)) return false;
    for (int k = 0; k < h.parts; ++k) {
        if (!h.out[k] || (uintptr_t)h.out[k] % 8 != 0) return false;
        if (h.gamma[k] && ((uintptr_t)h.gamma[k] % 16 != 0 || !h.rstd)) return false;
        if (h.gamma[k] && h.rope[k] &&
            (!h.tab || h.rope_dims <= 0 || h.rope_dims > kHeadDim || h.rope_dims % 8 != 0 || (uintptr_t)h.tab % 16 != 0))
            return false;
    }
    return true;
}

// Whether the attention dO epilogue fits this launch: one workgroup per tile, the staged epilogue
// with whole heads in each 16-lane group of a row (tiles of 64 or more columns), no accumulation,
// N = H x 64, M = B x Sq, 8-byte aligned bf16 rows.
bool attn_dot_ok(const DmaParams& p, int splits, int bn) {
    const AttnDot& a = p.ad;
    if (!a.doh || splits != 1 || !p.vec_epi || p.accumulate || bn < 64) return false;
    if (a.H <= 0 || a.Sq <= 0 || p.N != (int64_t)a.H * kHeadDim || p.M % a.Sq != 0 || p.M >= ((int64_t)1 << 31))
        return false;
    return a.o1 && a.o2 && a.dn1 && a.dn2 && (uintptr_t)a.doh % 8 == 0 && (uintptr_t)a.o1 % 8 == 0 &&
           (uintptr_t)a.o2 % 8 == 0;
}
// Whether the SwiGLU backward epilogue fits: one workgroup per tile, the staged epilogue, no
// accumulation, N = I (a multiple of 4), 8-byte aligned bf16 rows, a 16-byte aligned row scale.
bool swiglu_bwd_ok(const DmaParams& p, int splits) {
    const SwiBwd& b = p.sb;
    if (!b.du || !b.F || splits != 1 || !p.vec_epi || p.accumulate || p.N != b.I || b.I % 4 != 0) return false;
    return (uintptr_t)b.F % 8 == 0 && (uintptr_t)b.du % 8 == 0 && (!b.dsc || (uintptr_t)b.dsc % 16 == 0);
}
// Keep the backward epilogues this launch can run (then C is not written and *bwd_done is set);
// switch the others off, so that C is written for the caller's own kernels.
void settle_bwd_epilogues(DmaParams& p, int splits, int bn) {
    if (!p.ad.doh && !p.sb.du) return;
    if (p.ad.doh && !attn_dot_ok(p, splits, bn)) p.ad.doh = nullptr;
    if (p.sb.du && !swiglu_bwd_ok(p, splits)) p.sb.du = nullptr;
    if (p.ad.doh || p.sb.du) {
        if (p.bwd_done) *p.bwd_done = 1;
        p.C = nullptr;
    }
}

template <int BM, int BN, int WMW, int STAGES, bool BF16, int NW = 4, bool KN = false, int BQ = 0, bool HP = false>
void launch_dma(sa3k_ctx* ctx, DmaParams p) {
    const int64_t tiles = ceil_div(p.M + p.Mx, BM) * ceil_div(p.Nt, BN);
    const int64_t grid = ceil_div(tiles, 8) * 8;
    const int KT = (int)(p.K / (BF16 ? 64 : 32));
    // resident workgroups per CU: as many as the 160 KiB of LDS hold (or the context's override)
    constexpr int kLdsBytes = STAGES * (BM + BN) * kRow + 64;
    const int wg_per_cu = ctx->gemm_wg_per_cu > 0 ? ctx->gemm_wg_per_cu : std::max(1, (160 * 1024) / kLdsBytes);
    const int64_t slots = (int64_t)256 * wg_per_cu;
    static_assert((int64_t)256 * std::max(1, (160 * 1024) / kLdsBytes) * BM * BN <= kMaxSplitFloats,
                  "split partials of this tile family exceed kMaxSplitFloats");
    const int splits = split_count(ctx, tiles, slots, KT, &p.kps);
    p.ws = nullptr;
    p.counters = nullptr;
    {
        // main-segment byte extents for buffer descriptors (0 when they exceed 32-bit offsets)
        const int64_t eb = BF16 ? 2 : 4;
        auto extent = [&](int64_t rows, int64_t ld) -> uint32_t {
            const int64_t b = rows > 0 ? ((rows - 1) * ld + p.K) * eb : 0;
            return (b > 0 && b < ((int64_t)1 << 32)) ? (uint32_t)b : 0u;
        };
        p.a_bytes = extent(p.M, p.lda);
        p.ax_bytes = p.Mx > 0 ? extent(p.Mx, p.ldax) : 0u;
        p.b_bytes = extent(p.N, p.ldb);
        if (KN) {   // [K][ldb]: the whole matrix (the kernel addresses it through the descriptor only)
            const int64_t b = p.K * p.ldb * eb;
            p.b_bytes = b < ((int64_t)1 << 32) ? (uint32_t)b : 0u;
            SA3K_REQUIRE(p.b_bytes != 0 && p.a_bytes != 0 && (p.Mx == 0 || p.ax_bytes != 0),
                         "a [K][N] B operand needs buffer-addressable operands");
        }
        p.bx_bytes = p.Nx > 0 ? extent(p.Nx, p.ldbx) : 0u;
        if (KN && p.Nx > 0) {   // [K][Nx] extra columns, whole 64-column sub-tiles of the main ones
            SA3K_REQUIRE(p.N % 64 == 0 && p.Nx % 8 == 0 && p.Nx <= p.ldbx, "[K][N] extra columns need N % 64 == 0");
            const int64_t b = ((p.K - 1) * p.ldbx + p.Nx) * 2;
            p.bx_bytes = b < ((int64_t)1 << 32) ? (uint32_t)b : 0u;
            SA3K_REQUIRE(p.bx_bytes != 0, "[K][N] extra columns beyond a buffer descriptor's reach");
        }
        if (BQ == 2) {   // int8 quants (ldb bytes per row) and f16 block scales (ldbs per row)
            const int64_t qb = (p.N - 1) * p.ldb + p.K, sb = ((p.N - 1) * p.ldbs + p.K / 32) * 2;
            p.b_bytes = qb < ((int64_t)1 << 31) ? (uint32_t)qb : 0u;
            p.bs_bytes = sb < ((int64_t)1 << 31) ? (uint32_t)sb : 0u;
            SA3K_REQUIRE(p.bs_bytes != 0, "Q8_0 scales beyond a buffer descriptor's reach");
        }
        if (BQ != 0)
            SA3K_REQUIRE(p.a_bytes != 0 && p.b_bytes != 0 && p.Mx == 0 && p.Nx == 0,
                         "a decoded B operand needs buffer-addressable operands and no extra rows or columns");
        // the staged epilogue stores 4 columns at once: rows and vectors must be 16-byte (f32) /
        // 8-byte (bf16) aligned
        auto ok = [](const void* q, int64_t ld, int align) {
            return q == nullptr || (ld % 4 == 0 && (uintptr_t)q % (uintptr_t)align == 0);
        };
        p.nt_store = ctx->gemm_nt_store;
        p.vec_epi = p.N % 4 == 0 && p.Nt % 4 == 0 && ok(p.C, p.ldc, 16) && ok(p.U, p.ldu, 16) &&
                    ok(p.Ub, p.ldu, 8) && ok(p.Cb, p.ldcb, 8) && ok(p.Cx, p.ldcx, 16) && ok(p.Cbx, p.ldcx, 8) &&
                    ok(p.colscale, 4, 16) && ok(p.bias, 4, 16) && ok(p.Cbn, p.ldcn, 8);
    }
    settle_swiglu(p, BN, splits, KN, BQ);
    // the backward epilogues: only on the bf16 [K][N] instantiations (the merged dX products)
    constexpr bool kXE = BF16 && KN && BQ == 0 && !HP;
    if (!kXE) {
        p.ad.doh = nullptr;
        p.sb.du = nullptr;
    }
    settle_bwd_epilogues(p, splits, BN);
    if constexpr (HP) {
        if (!headprep_ok(p, splits)) {   // the caller prepares the heads: the plain instantiation
            p.hp.parts = 0;
            return launch_dma<BM, BN, WMW, STAGES, BF16, NW, KN, BQ, false>(ctx, p);
        }
        if (p.hp_done) *p.hp_done = 1;
        if (p.c_unfused_only) p.C = nullptr;
    }
    if (splits > 1) {
        p.ws = gemm_workspace_bytes(ctx, (size_t)splits * (size_t)(p.M + p.Mx) * (size_t)p.Nt * sizeof(float));
        if (use_fixup(ctx, (p.M + p.Mx) * p.Nt, tiles)) p.counters = stream_counters(ctx);
    }
    dim3 g((unsigned)grid, (unsigned)splits);
    {
        // profiled per kernel instantiation, with its algorithmic flops (padding excluded)
        static const std::string name = std::string("gemm_dma<") + std::to_string(BM) + "," + std::to_string(BN) + "," +
                                        std::to_string(WMW) + "," + std::to_string(STAGES) +
                                        (NW != 4 ? ",w" + std::to_string(NW) : std::string()) + (KN ? ",kn" : "") +
                                        (BQ == 1 ? ",f16b" : BQ == 2 ? ",q8b" : "") + (HP ? ",hp" : "") +
                                        (BF16 ? ",bf16>" : ",f32>");
        KernelScope ks(ctx, name.c_str(), 2.0 * (double)(p.M + p.Mx) * (double)p.Nt * (double)(p.K + p.K2));
        auto kern = gemm_dma_kernel<BM, BN, WMW, STAGES, BF16, NW, KN, BQ, HP>;
        if constexpr (kXE)
            if (p.ad.doh || p.sb.du) kern = gemm_dma_kernel<BM, BN, WMW, STAGES, BF16, NW, KN, BQ, HP, true>;
        launch_k(ctx, !(splits > 1 && !p.counters), kern, g, dim3(NW * 64), 0, p);
        SA3K_LAUNCHED();
    }
    if (splits > 1 && !p.counters) {
        KernelScope ks(ctx, "gemm_splitk_reduce");
        const int64_t items = p.vec_epi ? (p.M + p.Mx) * p.Nt / 4 : (p.M + p.Mx) * p.Nt;
        launch_k(ctx, true, gemm_dma_splitk_reduce, dim3((unsigned)ceil_div(items, kThreads)), dim3(kThreads), 0, p,
                 splits);
        SA3K_LAUNCHED();
    }
}

// Whether gemm_big_kernel can take this bf16 product: every extent addressable by a buffer
// descriptor, extra rows starting on an 8-row boundary, no in-kernel split reduction.
bool big_ok(const sa3k_ctx* ctx, const DmaParams& p) {
    auto extent = [&](int64_t rows, int64_t ld, int64_t k) -> int64_t { return rows > 0 ? ((rows - 1) * ld + k) * 2 : 0; };
    const int64_t lim = (int64_t)1 << 31;
    if (ctx->gemm_fixup != 0 || p.prescale) return false;
    if (extent(p.M, p.lda, p.K) >= lim || extent(p.N, p.ldb, p.K) >= lim) return false;
    if (p.b_kn && p.K * p.ldb * 2 >= lim) return false;
    if (p.Nx > 0 && (p.N % 8 != 0 || extent(p.Nx, p.ldbx, p.K) >= lim)) return false;
    if (p.b_kn && p.Nx > 0 && (p.N % 64 != 0 || p.Nx % 8 != 0 || (p.K - 1) * p.ldbx * 2 + p.Nx * 2 >= lim)) return false;
    if (p.Mx > 0 && (p.M % 8 != 0 || extent(p.Mx, p.ldax, p.K) >= lim)) return false;
    if (p.K2 > 0 && (extent(p.M, p.lda2, p.K2) >= lim || extent(p.N, p.ldb2, p.K2) >= lim ||
                     (p.Mx > 0 && extent(p.Mx, p.lda2x, p.K2) >= lim)))
        return false;
    return true;
}

// outputs allow the staged epilogue's 4-column stores: rows and vectors 16-byte (f32) / 8-byte
// (bf16) aligned
bool vec_epi_ok(const DmaParams& p) {
    auto ok = [](const void* q, int64_t ld, int align) {
        return q == nullptr || (ld % 4 == 0 && (uintptr_t)q % (uintptr_t)align == 0);
    };
    return p.N % 4 == 0 && p.Nt % 4 == 0 && ok(p.C, p.ldc, 16) && ok(p.U, p.ldu, 16) && ok(p.Ub, p.ldu, 8) &&
           ok(p.Cb, p.ldcb, 8) && ok(p.Cx, p.ldcx, 16) && ok(p.Cbx, p.ldcx, 8) && ok(p.colscale, 4, 16) &&
           ok(p.bias, 4, 16) && ok(p.Cbn, p.ldcn, 8);
}

void launch_big(sa3k_ctx* ctx, DmaParams p) {
    constexpr int BM = 256, BN = 256;
    const int64_t tiles = ceil_div(p.M + p.Mx, BM) * ceil_div(p.Nt, BN);
    const int64_t grid = ceil_div(tiles, 8) * 8;
    const int KT = (int)(p.K / 64);
    const int64_t slots = 256;   // one workgroup per CU (128 KiB of LDS)
    static_assert((int64_t)256 * 256 * 256 <= kMaxSplitFloats, "256 x 256 split partials exceed kMaxSplitFloats");
    const int splits = split_count(ctx, tiles, slots, KT, &p.kps);
    p.ws = nullptr;
    p.counters = nullptr;
    auto extent = [&](int64_t rows, int64_t ld) -> uint32_t { return rows > 0 ? (uint32_t)(((rows - 1) * ld + p.K) * 2) : 0u; };
    p.a_bytes = extent(p.M, p.lda);
    p.ax_bytes = extent(p.Mx, p.ldax);
    p.b_bytes = extent(p.N, p.ldb);
    p.bx_bytes = extent(p.Nx, p.ldbx);
    if (p.b_kn) p.b_bytes = (uint32_t)(p.K * p.ldb * 2);   // the whole [K][ldb] operand (big_ok: < 2 GiB)
    if (p.b_kn && p.Nx > 0) {   // [K][Nx] extra columns (big_ok: N % 64 == 0, within reach)
        SA3K_REQUIRE(p.N % 64 == 0 && p.Nx % 8 == 0 && p.Nx <= p.ldbx, "[K][N] extra columns need N % 64 == 0");
        p.bx_bytes = (uint32_t)(((p.K - 1) * p.ldbx + p.Nx) * 2);
    }
    p.nt_store = ctx->gemm_nt_store;
    p.vec_epi = 1;
    settle_swiglu(p, BN, splits, p.b_kn != 0, 0);
    if (!p.b_kn) {   // the backward epilogues: [K][N] instantiations only, as in launch_dma
        p.ad.doh = nullptr;
        p.sb.du = nullptr;
    }
    settle_bwd_epilogues(p, splits, BN);
    const bool xe = p.ad.doh || p.sb.du;
    if (splits > 1) p.ws = gemm_workspace_bytes(ctx, (size_t)splits * (size_t)(p.M + p.Mx) * (size_t)p.Nt * sizeof(float));
    {
        KernelScope ks(ctx, p.b_kn ? "gemm_big<256,256,kn,bf16>" : "gemm_big<256,256,bf16>",
                       2.0 * (double)(p.M + p.Mx) * (double)p.Nt * (double)(p.K + p.K2));
        // 16 waves of 64 x 64 (four per SIMD); option gemm_cfg 4: 8 waves of 64 x 128 (the DiT update
        // 32.90 against 33.08 ms on one box)
        const dim3 g((unsigned)grid, (unsigned)splits);
        if (ctx->gemm_cfg == 4) {
            if (p.b_kn) launch_k(ctx, splits == 1, xe ? gemm_big_kernel<true, 8, true> : gemm_big_kernel<true, 8>, g,
                                 dim3(512), 0, p);
            else launch_k(ctx, splits == 1, gemm_big_kernel<false, 8>, g, dim3(512), 0, p);
        } else {
            if (p.b_kn) launch_k(ctx, splits == 1, xe ? gemm_big_kernel<true, 16, true> : gemm_big_kernel<true, 16>, g,
                                 dim3(1024), 0, p);
            else launch_k(ctx, splits == 1, gemm_big_kernel<false, 16>, g, dim3(1024), 0, p);
        }
        SA3K_LAUNCHED();
    }
    if (splits > 1) {
        KernelScope ks(ctx, "gemm_splitk_reduce");
        const int64_t items = p.vec_epi ? (p.M + p.Mx) * p.Nt / 4 : (p.M + p.Mx) * p.Nt;
        launch_k(ctx, true, gemm_dma_splitk_reduce, dim3((unsigned)ceil_div(items, kThreads)), dim3(kThreads), 0, p,
                 splits);
        SA3K_LAUNCHED();
    }
}

// [K][N] B operands (bf16): the tiles of the default dispatch that have whole 64-column sub-tiles
void dispatch_dma_kn(sa3k_ctx* ctx, const DmaParams& p) {
    const int64_t Mt = p.M + p.Mx;
    if (use_big_tiles(ctx, Mt, p.N, p.K) && big_ok(ctx, p) && vec_epi_ok(p)) return launch_big(ctx, p);
    if (Mt <= 32) return launch_dma<32, 128, 1, 4, true, 4, true>(ctx, p);
    if (p.N <= 64) return launch_dma<128, 64, 4, 4, true, 4, true>(ctx, p);
    const int64_t tiles128 = ceil_div(Mt, 128) * ceil_div(p.N, 128);
    if (tiles128 < 384 && p.K < 4096 && ctx->gemm_small == 2) return launch_dma<64, 128, 1, 3, true, 4, true>(ctx, p);
    if (tiles128 < 384 && ctx->gemm_small == 4) return launch_dma<128, 128, 2, 3, true, 8, true>(ctx, p);
    if (ctx->gemm_cfg == 1) return launch_dma<128, 128, 2, 2, true, 4, true>(ctx, p);
    if (ctx->gemm_cfg == 4) return launch_dma<128, 256, 2, 3, true, 8, true>(ctx, p);
    return launch_dma<128, 256, 2, 3, true, 16, true>(ctx, p);
}

// B decoded from f16 / Q8_0 on its way into the MFMAs (bf16 A): the short-K small-grid tile of the
// bf16 dispatch, else 128 x 256 tiles with the 8 waves side by side along N (128 x 32 each), so
// every B fragment is decoded by one wave only (measured on MI355X, 2176 x 6144 x 1536 over Q8_0:
// 91.5 us against 107.5 us with 2 x 4 waves of 64 x 64, whose two wave rows decode each fragment);
// option gemm_dq 2 keeps the 2 x 4 layout. Both sum every output in the same order.
template <int BQ>
void dispatch_dma_dq(sa3k_ctx* ctx, const DmaParams& p) {
    const int64_t tiles128 = ceil_div(p.M, 128) * ceil_div(p.N, 128);
    // (decoded B: the 64 x 128 tile, whose four waves side by side along N decode each fragment once)
    if (tiles128 < 384 && p.K < 4096 && (ctx->gemm_small == 2 || ctx->gemm_small == 4))
        return launch_dma<64, 128, 1, 3, true, 4, false, BQ>(ctx, p);
    if (ctx->gemm_dq == 2) return launch_dma<128, 256, 2, 3, true, 8, false, BQ>(ctx, p);
    return launch_dma<128, 256, 1, 3, true, 8, false, BQ>(ctx, p);
}

template <bool BF16>
void dispatch_dma(sa3k_ctx* ctx, const DmaParams& p) {
    if constexpr (BF16) {
        // per-head q/k preparation: 128 x 256 tiles, the default for the attention projections
        // (falls back to the plain instantiation where headprep_ok refuses)
        if (p.hp.parts > 0 && p.bq == 0 && !p.b_kn) {
            if (ctx->gemm_cfg == 4) return launch_dma<128, 256, 2, 3, true, 8, false, 0, true>(ctx, p);
            return launch_dma<128, 256, 2, 3, true, 16, false, 0, true>(ctx, p);
        }
        if (p.bq == 1) return dispatch_dma_dq<1>(ctx, p);
        if (p.bq == 2) return dispatch_dma_dq<2>(ctx, p);
        if (p.b_kn) return dispatch_dma_kn(ctx, p);
        if (use_big_tiles(ctx, p.M + p.Mx, p.Nt, p.K) && big_ok(ctx, p) && vec_epi_ok(p)) return launch_big(ctx, p);
    }
    const int64_t Mt = p.M + p.Mx;
    if (Mt <= 32) return launch_dma<32, 128, 1, 4, BF16>(ctx, p);
    if (p.Nt <= 32) return launch_dma<128, 32, 4, 4, BF16>(ctx, p);
    if (p.Nt <= 64) return launch_dma<128, 64, 4, 4, BF16>(ctx, p);
    // Grids of 128x128 tiles that leave a quarter of the two-per-CU slots idle. bf16: no split, on
    // 128 x 128 tiles with eight waves in one workgroup per CU (three stages, 96 KiB), at any K
    // (measured on MI355X: 2176 x 1536 x 1536 21.4 us against 23.6 us on 64 x 128 tiles and 31.1 us
    // on the default tile split over K; 2176 x 1536 x 6144 67.7 against 71.1 us split over K; the
    // DiT update 34.56 against 35.16 ms with the short-K products alone, then 33.66 against 33.97 ms
    // with the long-K ones too). f32 with a short K: 64 x 128 tiles, no split.
    const int64_t tiles128 = ceil_div(Mt, 128) * ceil_div(p.Nt, 128);
    if constexpr (BF16)
        if (tiles128 < 384 && ctx->gemm_small == 4) return launch_dma<128, 128, 2, 3, true, 8>(ctx, p);
    if (tiles128 < 384 && p.K < (BF16 ? 4096 : 2048)) {
        switch (ctx->gemm_small) {
            case 1: return launch_dma<64, 128, 2, 2, BF16>(ctx, p);
            case 2: case 4: return launch_dma<64, 128, 1, 3, BF16>(ctx, p);
            case 3: return launch_dma<128, 64, 2, 2, BF16>(ctx, p);
            default: break;
        }
    }
    // bf16: 128 x 256 tiles, three stages in 144 KiB of LDS (one workgroup per CU), 16 waves of
    // 64 x 32 (four per SIMD, to hide the DMA and LDS latency behind each other's MFMAs). Against
    // two 128 x 128 workgroups per CU the tile moves a quarter fewer operand bytes per flop through
    // the CU's vector-memory path, which the MFMA rate otherwise saturates (measured on MI355X at
    // 2176 rows, 8 waves: QKV 2176 x 7680 x 1536 58.2 vs 64.7 us, 2176 x 3072 x 1536 27.4 vs
    // 31.0 us, the split-K products 2176 x 1536 x 6144 / 7680 / 12288 53.4 / 63.5 / 93.5 vs
    // 59.4 / 70.7 / 102.2 us); 16 waves against 8 (option gemm_cfg 4): 2176 x 7680 x 1536 with f32
    // output 76.7 vs 86.6 us, the DiT update 34.57 vs 35.00 ms.
    switch (ctx->gemm_cfg) {
        case 1: return launch_dma<128, 128, 2, 2, BF16>(ctx, p);    // 64 KiB LDS: two workgroups per CU
        case 4: return launch_dma<128, 256, 2, 3, BF16, 8>(ctx, p);
        case 7: return launch_dma<128, 256, 2, 2, BF16, 8>(ctx, p);
        default:
            if constexpr (BF16) return launch_dma<128, 256, 2, 3, true, 16>(ctx, p);
            else return launch_dma<128, 128, 2, 2, false>(ctx, p);
    }
}

// Rounds of resident workgroups a bf16 DMA GEMM of Mt x Nt x K takes under the dispatch above
// (the tile and split choices, ignoring operand alignment): splits x tiles / slots, rounded up.
int64_t dma_rounds(const sa3k_ctx* ctx, int64_t Mt, int64_t Nt, int64_t K) {
    const int KT = (int)(K / 64);
    auto rounds = [&](int64_t tiles, int64_t slots) {
        return ceil_div(tiles * split_count(ctx, tiles, slots, KT, nullptr), slots);
    };
    if (use_big_tiles(ctx, Mt, Nt, K)) return rounds(ceil_div(Mt, 256) * ceil_div(Nt, 256), 256);
    if (Mt <= 32 || Nt <= 64) return 1;
    const int64_t tiles128 = ceil_div(Mt, 128) * ceil_div(Nt, 128);
    if (tiles128 < 384 && K < 4096 && ctx->gemm_small == 2) return rounds(ceil_div(Mt, 64) * ceil_div(Nt, 128), 512);
    if (tiles128 < 384 && ctx->gemm_small == 4) return rounds(tiles128, 256);
    if (ctx->gemm_cfg == 1) return rounds(tiles128, 512);
    return rounds(ceil_div(Mt, 128) * ceil_div(Nt, 256), 256);
}

}  // namespace

// Whether Nx extra output columns ride on a bf16 Mt x N x K product without costing it another
// round of workgroups (their tiles fill slots the product leaves idle).
bool gemm_extra_cols_free(const sa3k_ctx* ctx, int64_t Mt, int64_t N, int64_t K, int64_t Nx) {
    return dma_rounds(ctx, Mt, N + Nx, K) <= dma_rounds(ctx, Mt, N, K);
}

void gemm_run_dma(sa3k_ctx* ctx, const GemmDesc& d) {
    DmaParams p{d.A, d.lda, d.B, d.ldb, d.A2, d.lda2, d.B2, d.ldb2, d.K2, d.M, d.N, d.K, d.alpha,
                d.colscale, d.bias, d.C, d.ldc, d.accumulate, d.Cb, d.ldcb, d.U, d.Ub, d.ldu,
                d.Mx, d.Ax, d.ldax, d.A2x, d.lda2x, d.Cx, d.ldcx, d.accumulate_x, d.Cbx, nullptr, 0, ctx->zero_page};
    p.prescale = d.prescale;
    p.Nx = d.Nx;
    p.Nt = d.N + d.Nx;
    p.Bx = d.Bx; p.ldbx = d.ldbx;
    p.alpha_x = d.alpha_x;
    p.Cbn = d.Cbn; p.ldcn = d.ldcn;
    p.bx_bytes = 0;
    p.b_kn = d.b_kn;
    p.bq = d.b_src == SRC_F16 ? 1 : d.b_src == SRC_Q8 ? 2 : 0;
    p.Bs = d.Bs; p.ldbs = d.ldbs;
    p.bs_bytes = 0;
    p.sw_half = d.sw_half; p.sw_g = d.sw_g; p.sw_ldg = d.sw_ldg; p.sw_done = d.sw_done;
    p.hp = d.hp; p.hp_done = d.hp_done; p.c_unfused_only = d.c_unfused_only;
    p.ad = d.ad; p.sb = d.sb; p.bwd_done = d.bwd_done;
    p.prio = ctx->gemm_prio;
    if (d.prec == SA3K_PREC_BF16) dispatch_dma<true>(ctx, p);
    else dispatch_dma<false>(ctx, p);
}

}  // namespace sa3k
