// Flat-HTRC attention kernels for MI355X (gfx950, CDNA4), and their C-ABI launchers.
//
// Pipeline of one layer call (every kernel takes a head index in grid.z / grid.y, so all
// heads of a layer go in one launch):
//   pack_q    q rows -> tile centres mu, q8/sq, dq8/sdq          (HBM-bound)
//   pack_k    k      -> k8/ks                                     (HBM-bound)
//   stats     mu, K, V -> per (tile, leaf) g8/sg, vb, lz          (bf16 MFMA, HBM writes)
//   select    dq8, g8 -> SEL[t, l]                                (int8 MFMA)
//   topk      SEL -> idx (ascending), excl                        (LDS radix select)
//   tile      far (g8, vb) + near (k8, v) online softmax          (int8 + bf16 MFMA)
//   merge     split partials -> out, logZ
//
// MFMA conventions (16x16xK): lane l supplies A[m = l%16][k-set(l/16)] and
// B[k-set(l/16)][n = l%16]; C[m = 4*(l/16) + i][n = l%16] sits in item i of lane l.
// Every product below is arranged as C^T = A(keys/dims) * B(query rows or centres), so the
// query row (or tile centre) of a C element is always lane%16 and the online-softmax
// statistics of a row never leave its four lanes.
//
// PV-type operands (eight k-items = two runs of four consecutive keys at one column) are
// read from row-major data staged in LDS with the gfx950 transposing read (lds_read_tr16).
#include "common.h"

#include <stdio.h>
#include <string.h>
#include <atomic>
#include <mutex>

using namespace htrc;

// ---------------------------------------------------------------------------------------------
// pack_q: one workgroup per (tile, head).  Tile centre = sequential fp32 sum over the real
// rows / row count (h3/htrc_flat.py:142-156); then per padded row the int8 of q and of
// q - mu with per-row scales (h3/htrc_flat_triton.py:104-117).  Each 16-lane group of a wave
// quantises one row (8 values per lane, row max by DPP), 16-byte loads and 8-byte stores.
// ---------------------------------------------------------------------------------------------
// Eight int8 codes, as int32 in [-128, 127], packed little-endian.
__device__ __forceinline__ u32x2 pack8_i8(const int (&c)[8]) {
    return u32x2{pack4_i8(c[0], c[1], c[2], c[3]), pack4_i8(c[4], c[5], c[6], c[7])};
}

// Query row of operator row p of head h under an optional permutation (order="kmeans"); entries
// are clamped to the head, so a malformed permutation cannot address outside it.
__device__ __forceinline__ int64_t perm_row(const int32_t* perm, int64_t h, int64_t nq, int64_t p) {
    if (!perm) return p;
    const int64_t r = perm[h * nq + p];
    return r < 0 ? 0 : (r >= nq ? nq - 1 : r);
}

// Shared centres of tile groups (h3/htrc_flat.py:223-229): mu_g is the mean of the G * tile
// rows of tiles gG .. gG + G - 1, where tiles past the last repeat the last tile and rows past
// the last query repeat the last query (the reference pads the tiles, then averages every
// padded row).  One thread per dim: sequential fp32 sum over the group's rows in order, then
// one IEEE division.
template <bool IN_BF16>
__global__ __launch_bounds__(128) void group_centres_kernel(const void* __restrict__ qin, int64_t nq, int nt,
                                                            int tile, int group, int ng,
                                                            const int32_t* __restrict__ perm, float* __restrict__ mu) {
    const int g = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
    const int64_t qbase = (int64_t)h * nq * D;
    const int rows = group * tile;
    float s = 0.0f;
    for (int j0 = 0; j0 < rows; j0 += 8) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = j0 + u;
            const int t = min(g * group + j / tile, nt - 1);
            const int64_t pp = min((int64_t)t * tile + j % tile, nq - 1);
            const int64_t p = perm_row(perm, h, nq, pp);
            x[u] = IN_BF16 ? bf2f(((const uint16_t*)qin)[qbase + p * D + i]) : ((const float*)qin)[qbase + p * D + i];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) s = __fadd_rn(s, x[u]);
    }
    mu[((int64_t)h * ng + g) * D + i] = __fdiv_rn(s, (float)rows);
}

// One workgroup per tile of `tile` (32 or 64) rows.  group == 1: the tile's centre over its
// real rows is computed here and written to mu; group > 1: the group's centre is read from mu
// (group_centres_kernel).  perm (optional): row p of the operator is query perm[p]
// (order="kmeans").
// QM = 0: row int8 of q and q - mu (q8 / sq, dq8 / sdq).  QM = 1, 2: the 16-bit operands of the
// reference's bf16 and fp8 state stores: q in bf16 (q8 holds uint16 rows, sq unused) and q - mu in
// bf16 (QM = 1) or fp16 (QM = 2) (h3/htrc_flat_triton.py:104-108, dqb / dqh; dq8 holds them).
template <bool IN_BF16, int QM = 0>
__global__ __launch_bounds__(256) void pack_q_kernel(const void* __restrict__ qin, int64_t nq, int nt, int tile,
                                                     int group, int ng, const int32_t* __restrict__ perm,
                                                     float* __restrict__ mu, int8_t* __restrict__ q8,
                                                     float* __restrict__ sq, int8_t* __restrict__ dq8,
                                                     float* __restrict__ sdq) {
    // the tile's rows as loaded (bf16 rows padded by 16 bytes, fp32 rows by 16 bytes): 17 KB for
    // bf16 input, so eight workgroups share a CU and hide each other's load latency
    using TQ = typename std::conditional<IN_BF16, uint16_t, float>::type;
    constexpr int TQP = IN_BF16 ? 8 : 4;
    __shared__ __align__(16) TQ tq[TILE][D + TQP];
    __shared__ __align__(16) float smu[D];
    auto tq_at = [&](int r, int c) { return IN_BF16 ? bf2f(tq[r][c]) : (float)tq[r][c]; };
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int64_t r0 = (int64_t)t * tile;
    const int nr = (int)(nq - r0 < tile ? nq - r0 : tile);
    const int64_t qbase = (int64_t)h * nq * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {               // 8 consecutive values per thread and chunk
        if (16 * j >= tile) break;              // chunk j holds rows 16j .. 16j + 15
        const int c = tid + 256 * j, r = c >> 4, c8 = (c & 15) * 8;
        const int64_t pr = r0 + r < nq ? r0 + r : nq - 1;                      // pad rows repeat the last row
        const int64_t src = qbase + perm_row(perm, h, nq, pr) * D + c8;
        if constexpr (IN_BF16) {
            *(u32x4*)&tq[r][c8] = __builtin_nontemporal_load((const u32x4*)((const uint16_t*)qin + src));
        } else {
            *(f32x4*)&tq[r][c8] = __builtin_nontemporal_load((const f32x4*)((const float*)qin + src));
            *(f32x4*)&tq[r][c8 + 4] = __builtin_nontemporal_load((const f32x4*)((const float*)qin + src + 4));
        }
    }
    __syncthreads();
    const int64_t tg = (int64_t)h * nt + t;
    if (tid < D) {
        if (group == 1) {
            float s = 0.0f;
            for (int r = 0; r < nr; ++r) s = __fadd_rn(s, tq_at(r, tid));
            const float m = __fdiv_rn(s, (float)nr);
            smu[tid] = m;
            mu[tg * D + tid] = m;
        } else {
            smu[tid] = mu[((int64_t)h * ng + t / group) * D + tid];
        }
    }
    __syncthreads();
    const int w = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
    if (16 * w >= tile) return;                    // wave w packs rows 16w .. 16w + 15
    float m[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) m[e] = smu[8 * i + e];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int r = 16 * w + 4 * it + g;         // row of this 16-lane group
        float x[8], d[8], aq = 0.0f, ad = 0.0f;
        if constexpr (IN_BF16) {
            const u32x4 u = *(const u32x4*)&tq[r][8 * i];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = __uint_as_float(w4[e] << 16);
                x[2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = tq[r][8 * i + e];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            d[e] = __fsub_rn(x[e], m[e]);
            aq = fmaxf(aq, fabsf(x[e]));
            ad = fmaxf(ad, fabsf(d[e]));
        }
        const int64_t p = tg * tile + r;
        if constexpr (QM != 0) {
            uint32_t uq[4], ud[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uq[e] = pack2bf(x[2 * e], x[2 * e + 1]);
                ud[e] = QM == 1 ? pack2bf(d[2 * e], d[2 * e + 1]) : pack2h(d[2 * e], d[2 * e + 1]);
            }
            *(u32x4*)((uint16_t*)q8 + p * D + 8 * i) = u32x4{uq[0], uq[1], uq[2], uq[3]};
            *(u32x4*)((uint16_t*)dq8 + p * D + 8 * i) = u32x4{ud[0], ud[1], ud[2], ud[3]};
            continue;
        }
        const float s1 = row_scale(col_max(aq), 1e-20f), s2 = row_scale(col_max(ad), 1e-20f);
        const float y1 = __fdiv_rn(1.0f, s1), y2 = __fdiv_rn(1.0f, s2);
        int cq[8], cd[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            cq[e] = round_away(div_by(x[e], s1, y1));
            cd[e] = round_away(div_by(d[e], s2, y2));
        }
        // non-temporal: the rows are next read only after the statistics have streamed the whole
        // state through the caches (pack_q 3% faster alone)
        __builtin_nontemporal_store(pack8_i8(cq), (u32x2*)(q8 + p * D + 8 * i));
        __builtin_nontemporal_store(pack8_i8(cd), (u32x2*)(dq8 + p * D + 8 * i));
        if (i == 0) {
            sq[p] = s1;
            sdq[p] = s2;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// pack_k: one workgroup per 64 key rows of a head; each 16-lane group quantises one row
// (8 values per lane, row max by DPP).  k8/ks per row (h3/htrc_flat.py:216-218, round half
// to even).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_k_kernel(const uint16_t* __restrict__ k, int64_t nk,
                                                     int8_t* __restrict__ k8, float* __restrict__ ks) {
    const int h = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, i = lane & 15;
    const int64_t base = (int64_t)h * nk;
    // the four rows' loads are issued together, then each row is quantised and stored
    u32x4 ld[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int64_t r = (int64_t)blockIdx.x * 64 + 16 * w + 4 * it + g;
        ld[it] = r < nk ? __builtin_nontemporal_load((const u32x4*)(k + (base + r) * D + 8 * i)) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int64_t r = (int64_t)blockIdx.x * 64 + 16 * w + 4 * it + g;
        if (r >= nk) break;                       // nk % 16 == 0: whole 16-lane groups leave together
        const u32x4 u = ld[it];
        const float x[8] = {bf2f(u.x & 0xffffu), bf2f(u.x >> 16), bf2f(u.y & 0xffffu), bf2f(u.y >> 16),
                            bf2f(u.z & 0xffffu), bf2f(u.z >> 16), bf2f(u.w & 0xffffu), bf2f(u.w >> 16)};
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(x[e]));
        const float sc = row_scale(col_max(a), 1e-20f);
        const float y = __fdiv_rn(1.0f, sc);
        int c[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) c[e] = round_even_clamp(div_by(x[e], sc, y));
        *(u32x2*)(k8 + (base + r) * D + 8 * i) = pack8_i8(c);
        if (i == 0) ks[base + r] = sc;
    }
}

// ---------------------------------------------------------------------------------------------
// stats: leaf statistics at the tile centres (h3/htrc_flat_triton.py:41-85).  A workgroup
// holds a few leaves of one head and sweeps the head's centres, 16 per wave.  Per leaf:
//   a^T = K_l mu^T                      fp16 MFMA, mu in two fp16 terms (22 bits)
//   e = exp(a - max) per centre (lane%16 = centre), z = sum e
//   g^T = K_l^T w^T, vb^T = V_l^T w^T   w = e / z in two fp16 terms (g = scale * K_l^T w^T;
//                                        K, V exact in fp16 after a power-of-two scale)
// The leaves' K and V rows are staged in LDS as fp16 (XOR-swizzled 16-byte chunks); the QK
// operand is a plain 16-byte read, the PV-type operands come from the same rows through
// transposing reads.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }

// One direct global->LDS load: 16 bytes per lane from src to LDS address lds + lane * 16 (lds
// wave-uniform; it goes to M0).  Issued as inline asm on purpose: the compiler's wait-count
// pass treats every LDS DMA in flight as aliasing every later LDS read and puts a vmcnt(0)
// before it, which would serialise each ring slot with the loads issued for the slots after
// it.  The kernels order their LDS reads after the DMA themselves, with wait_vmcnt<N>.
// NT: non-temporal (the data is read once: it should not displace cached lines others reuse).
template <bool NT = false>
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                     : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                     : : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// The same load from a wave-uniform base (kept in SGPRs) plus a 32-bit per-lane byte offset
// voff.  (No instruction offset: on these loads it moves the LDS destination as well.)
template <bool NT = false>
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    // readfirstlane returns int: widen each half through uint32_t so the low half is not
    // sign-extended into the high one
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                     : : "v"(voff), "s"(bs), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                     : : "v"(voff), "s"(bs), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// Wave-uniform 64-bit address p - shift in an SGPR pair.
__device__ __forceinline__ uint64_t sbase(const void* p, uint32_t shift = 0) {
    const uint64_t b = (uint64_t)(uintptr_t)p - shift;
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
}

// Direct global->LDS loads sharing one M0 (= LDS address lds): load i writes LDS lds + 1024 i
// (+ lane * 16) from b_i + v_i + 1024 i.  The instruction offset moves the global and the LDS
// address alike (checked on gfx950), so callers pass base i already lowered by 1024 i.
template <bool NT = false>
__device__ __forceinline__ void dma_x2(uint64_t b0, uint32_t v0, uint64_t b1, uint32_t v1, uint32_t lds) {
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %4\n\ts_nop 0\n\t"
                     "global_load_lds_dwordx4 %0, %2 nt\n\t"
                     "global_load_lds_dwordx4 %1, %3 offset:1024 nt"
                     : : "v"(v0), "v"(v1), "s"(b0), "s"(b1), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %4\n\ts_nop 0\n\t"
                     "global_load_lds_dwordx4 %0, %2\n\t"
                     "global_load_lds_dwordx4 %1, %3 offset:1024"
                     : : "v"(v0), "v"(v1), "s"(b0), "s"(b1), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
template <bool NT = false>
__device__ __forceinline__ void dma_x4(uint64_t b0, uint32_t v0, uint64_t b1, uint32_t v1, uint64_t b2, uint32_t v2,
                                       uint64_t b3, uint32_t v3, uint32_t lds) {
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %8\n\ts_nop 0\n\t"
                     "global_load_lds_dwordx4 %0, %4 nt\n\t"
                     "global_load_lds_dwordx4 %1, %5 offset:1024 nt\n\t"
                     "global_load_lds_dwordx4 %2, %6 offset:2048 nt\n\t"
                     "global_load_lds_dwordx4 %3, %7 offset:3072 nt"
                     : : "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(b0), "s"(b1), "s"(b2), "s"(b3),
                       "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %8\n\ts_nop 0\n\t"
                     "global_load_lds_dwordx4 %0, %4\n\t"
                     "global_load_lds_dwordx4 %1, %5 offset:1024\n\t"
                     "global_load_lds_dwordx4 %2, %6 offset:2048\n\t"
                     "global_load_lds_dwordx4 %3, %7 offset:3072"
                     : : "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(b0), "s"(b1), "s"(b2), "s"(b3),
                       "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// s_waitcnt vmcnt(N): at most N vector-memory operations of this wave still in flight (they
// complete in issue order).  The memory clobber keeps the compiler from moving LDS reads of a
// DMA'd slot above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Operands loaded from global memory before a DMA loop: consuming them here makes the compiler
// wait for those loads before the loop's first DMA is issued (its own wait inside the loop would
// otherwise also drain the DMAs, which it cannot see).
__device__ __forceinline__ void settle(const i32x4 (&b)[4][2], const float (&s)[4]) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) asm volatile("" : : "v"(b[rb][0]), "v"(b[rb][1]), "v"(s[rb]));
}

// Exponent t of the power of two that brings a leaf's largest magnitude m into [2^14, 2^15)
// (m 2^-t; floored at -24, so rows of tiny values are raised by at most 2^24): every bf16 value
// of the leaf then converts to fp16 exactly unless it is below m 2^-28, and none overflows.
__device__ __forceinline__ int f16_exp(float m) {
    const int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;
    return e - 14 < -24 ? -24 : e - 14;
}

// The NL leaves [l0, l0 + NL) of K and V (rows of LEAF keys; leaves from lr on are padding and
// not loaded) as fp16 in LDS, each leaf's K and V scaled by its own power of two 2^-t (f16_exp of
// the matrix's largest |value| in the leaf); the exponents come back in tk, tv (wave-uniform).
// Layout per leaf (LEAF_BYTES = 32 LEAF 16): LDS chunk s = 256 j + tid holds the 16-byte chunk
// (s % 16) ^ swz(row) of row (s / 16) % LEAF of K (the first 16 LEAF chunks) or V.  Thread tid
// loads those chunks itself (16-byte global loads), so its rows are r_j + 4 w + lane / 16 with
// r_j = 16 j mod LEAF.  Two barriers: after the per-wave maxima, after the fp16 rows.
template <int LEAF, int NL>
__device__ __forceinline__ void stage_leaves_f16(const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                                                 int64_t key0, int nreal, char* lds, float (*lmax)[2][4],
                                                 int (&tk)[NL], int (&tv)[NL]) {
    constexpr int NJ = 32 * LEAF / 256;         // 16-byte chunks per thread and leaf (K: j < NJ / 2)
    constexpr int LEAF_BYTES = 32 * LEAF * 16;
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int rw = 4 * w + (lane >> 4);
    const int cg = (lane & 15) ^ swz(rw & 15);
    u32x4 ch[NL][NJ];
#pragma unroll
    for (int li = 0; li < NL; ++li) {
        us2 mk = {0, 0}, mv = {0, 0};
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint16_t* src = (j < NJ / 2 ? K : V) + (key0 + (int64_t)li * LEAF + (16 * j) % LEAF + rw) * D + 8 * cg;
            ch[li][j] = li < nreal ? *(const u32x4*)src : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const us2 x = __builtin_bit_cast(us2, ch[li][j][e] & 0x7fff7fffu);    // |bf16| bits order as integers
                if (j < NJ / 2) mk = __builtin_elementwise_max(mk, x); else mv = __builtin_elementwise_max(mv, x);
            }
        }
        const float fk = wave_max(bf2f(mk.x > mk.y ? mk.x : mk.y)), fv = wave_max(bf2f(mv.x > mv.y ? mv.x : mv.y));
        if (lane == 0) {
            lmax[li][0][w] = fk;
            lmax[li][1][w] = fv;
        }
    }
    __syncthreads();
#pragma unroll
    for (int li = 0; li < NL; ++li) {
        tk[li] = __builtin_amdgcn_readfirstlane(
            f16_exp(fmaxf(fmaxf(lmax[li][0][0], lmax[li][0][1]), fmaxf(lmax[li][0][2], lmax[li][0][3]))));
        tv[li] = __builtin_amdgcn_readfirstlane(
            f16_exp(fmaxf(fmaxf(lmax[li][1][0], lmax[li][1][1]), fmaxf(lmax[li][1][2], lmax[li][1][3]))));
        if (li >= nreal) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int t = j < NJ / 2 ? -tk[li] : -tv[li];
            const u32x4 u = ch[li][j];
            const u32x4 hv = {pack2h(ldexpf(bf2f(u.x & 0xffffu), t), ldexpf(bf2f(u.x >> 16), t)),
                              pack2h(ldexpf(bf2f(u.y & 0xffffu), t), ldexpf(bf2f(u.y >> 16), t)),
                              pack2h(ldexpf(bf2f(u.z & 0xffffu), t), ldexpf(bf2f(u.z >> 16), t)),
                              pack2h(ldexpf(bf2f(u.w & 0xffffu), t), ldexpf(bf2f(u.w >> 16), t))};
            *(u32x4*)(lds + li * LEAF_BYTES + (256 * j + tid) * 16) = hv;
        }
    }
    __syncthreads();
}

// PV-type operand half from swizzled LDS rows: keys rbase + 4grp + j (j = 0..3) at column
// 16db + lane%16.
__device__ __forceinline__ uint32_t tr_offset(int rbase, int db, int lane) {
    const int L = lane & 15, grp = lane >> 4;
    const int row = rbase + 4 * grp + (L >> 2);
    const int c = 2 * db + ((L & 3) >> 1);
    return (uint32_t)((row * 16 + (c ^ swz(row))) * 16 + 8 * (L & 1));
}
// The same read at LDS byte address a (an offset from tr_offset plus the rows' base): keys 16 on
// (rbase + 16) share the lane's swizzle (swz looks at the row's low four bits), so a caller
// adds 4096 for them, and a ring slot's byte offset, as constants the read takes as immediates.
__device__ __forceinline__ u32x2 tr_read(uint32_t a) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a);
    return __builtin_bit_cast(u32x2, v);
}
__device__ __forceinline__ u32x2 tr_operand(const char* rows, int rbase, int db, int lane) {
    const int L = lane & 15, grp = lane >> 4;
    const int row = rbase + 4 * grp + (L >> 2);
    const int c = 2 * db + ((L & 3) >> 1);
    return lds_read_tr16(rows + (row * 16 + (c ^ swz(row))) * 16 + 8 * (L & 1));
}

// OCP e4m3 (e4m3fn) code of x rounded to nearest even, |x| saturated at 448 (the largest
// finite value; the state scales keep |x| <= 448): below 2^-6 the subnormal grid m * 2^-9,
// above it the mantissa rounded to 3 bits in the float's bit pattern.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t sgn = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = fminf(fabsf(x), 448.0f);
    uint32_t c;
    if (a < 0.015625f) {
        c = (uint32_t)rintf(__fmul_rn(a, 512.0f));                 // 0 .. 8 (8: the smallest normal)
    } else {
        const uint32_t b = __float_as_uint(a);
        const uint32_t r = (b + 0x7ffffu + ((b >> 20) & 1u)) & 0xfff00000u;
        c = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
    }
    return sgn | c;
}

// e4m3 codes of x_i * c packed little-endian.
__device__ __forceinline__ uint32_t quant4_e4m3(f32x4 x, float c) {
    return f32_to_e4m3(__fmul_rn(x[0], c)) | (f32_to_e4m3(__fmul_rn(x[1], c)) << 8) |
           (f32_to_e4m3(__fmul_rn(x[2], c)) << 16) | (f32_to_e4m3(__fmul_rn(x[3], c)) << 24);
}

// The same codes from gfx950's conversion instruction (v_cvt_pk_fp8_f32: OCP e4m3, round to
// nearest even), two values per instruction.  It matches f32_to_e4m3 on every input with
// |x| < 464 (htrc_selftest_f32_e4m3 checks code values, ties, their neighbours, subnormals and
// random values on the device); the state scales keep |x c| <= 448 (1 + 2^-22).
__device__ __forceinline__ uint32_t quant4_e4m3_cvt(f32x4 x, float c) {
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(__fmul_rn(x[0], c), __fmul_rn(x[1], c), 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(__fmul_rn(x[2], c), __fmul_rn(x[3], c), r, true);
    return (uint32_t)r;
}

// int8 codes of x_i * c rounded half away from zero, packed little-endian: trunc(x c +
// copysign(0.5, x)) (h3/htrc_flat_triton.py:77-79: where(x >= 0, x + 0.5, x - 0.5) and a
// truncating int8 cast; 0.49999997 -> 1 as there), with x c +- 1/2 taken in one FMA (c > 0, so
// the sign is x's): against rounding x c first this differs only where x c lies within an ulp
// of a half-integer, and saves an instruction per code.  copysign is one bit select; v_cvt_i32_f32
// truncates, and its SDWA form writes the low byte of each code (the two's-complement int8) into
// byte i of the packed word in place.
__device__ __forceinline__ uint32_t quant4(f32x4 x, float c) {
    float z[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        z[i] = __fmaf_rn(x[i], c, __uint_as_float((__float_as_uint(x[i]) & 0x80000000u) | 0x3f000000u));
    uint32_t u = (uint32_t)(int)z[0];
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(u) : "v"(z[1]));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(u) : "v"(z[2]));
    asm("v_cvt_i32_f32_sdwa %0, %1 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(u) : "v"(z[3]));
    return u;
}

// Precomputed centre operands of the statistics kernel: per centre row of the window, its
// exponent smu (its largest |value| times 2^smu in [2^14, 2^15), smu in [-64, 64]) and the two fp16
// terms hi + lo of every dim times 2^smu (TF32: of the dim rounded to TF32 first, lo then 0), the
// same words stats_ls_kernel's in-kernel split makes.  Row: hi[128] | lo[128] | smu (int32) | pad.
constexpr int MUT_ROW = 2 * D + 8;
template <bool TF32>
__global__ __launch_bounds__(64) void centre_terms_kernel(const float* __restrict__ mu, int64_t mu_stride, int64_t c0,
                                                          int cn, uint16_t* __restrict__ mut) {
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const float* src = mu + ((int64_t)h * mu_stride + c0 + t) * D;
    const float x0 = src[2 * lane], x1 = src[2 * lane + 1];
    const float mx = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
    const int e = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 127;
    const int sm = 14 - e < -64 ? -64 : (14 - e > 64 ? 64 : 14 - e);
    const float y0 = ldexpf(TF32 ? tf32_rna(x0) : x0, sm), y1 = ldexpf(TF32 ? tf32_rna(x1) : x1, sm);
    const uint32_t hi = pack2h(y0, y1);
    const uint32_t lo = pack2h(sub_h_lo(y0, hi), sub_h_hi(y1, hi));
    uint16_t* row = mut + ((int64_t)h * cn + t) * MUT_ROW;
    *(uint32_t*)(row + 2 * lane) = hi;
    *(uint32_t*)(row + D + 2 * lane) = lo;
    if (lane == 0) *(int*)(row + 2 * D) = sm;
}

// Leaf statistics at the tile centres (h3/htrc_flat_triton.py:41-85), per (centre, leaf): the
// logits a = (mu . k) scale, lz = max + log sum exp, w = softmax, g = (w K) scale, vb = w V, by
// fp16 MFMA on fp32-accurate operands: K and V exact in fp16 (each leaf scaled by a power of
// two, stage_leaves_f16), mu and w as two fp16 terms hi + lo (22 bits; mu of each centre scaled
// by a power of two into [2^14, 2^15), w by 2^14, so lo keeps its bits: products exact, fp32
// sums).  Every power of two is taken out again exactly where the reference's scale enters
// (one rounding per value, as there).
// STORE 0: g int8 with row scale sg, vb bf16 (the production I8 store, :73-80);
// STORE 1: g and vb bf16, no scales (store="bf16", :82-83);
// STORE 2: g and vb as e4m3 codes of x / s with row scales s = max(max|x| * fp32(1/448), 1e-30)
// (sg, sv; store="fp8", :65-72); vb then holds bytes.
// Leaf-stationary schedule: a workgroup of four waves stages the K / V of NL leaves
// in LDS once (NL * LEAF = 128 keys, 64 KB of fp16), then each wave sweeps its share of the launch's
// centres, 16 at a time, through those leaves: every leaf's K / V leaves HBM once, and the loop
// has no barrier and no load wait for K / V.  The centres of the next group of 16 are loaded
// into registers while the current group is computed.  Its state rows are stored as soon as
// they are quantised; sg / lz (sv) of the NL leaves are NL contiguous floats per centre.
// ncs: the centre groups of a head are dealt over ncs workgroups (small layers).
template <int LEAF, int STORE, int NL, bool TF32 = false, bool MUT = false>
__global__ __launch_bounds__(256, 2) void stats_ls_kernel(const float* __restrict__ mu, const uint16_t* __restrict__ mut,
                                                          int64_t mu_stride,
                                                          int64_t c0, int nt, const uint16_t* __restrict__ k,
                                                          const uint16_t* __restrict__ v, int64_t nk, int nb,
                                                          int nb_pad, int ncs, float scale, int8_t* __restrict__ g8,
                                                          float* __restrict__ sg, uint16_t* __restrict__ vb,
                                                          float* __restrict__ sv, float* __restrict__ lz) {
    constexpr int KB = LEAF / 16;
    constexpr int KK = (LEAF + 31) / 32;
    constexpr int LEAF_BYTES = 32 * LEAF * 16;
    constexpr bool FP8 = STORE == 2, BF16 = STORE == 1, F32 = STORE == 3, HAS_SG = STORE == 0 || STORE == 2;
    static_assert(NL * LEAF_BYTES <= 65536 && (NL == 1 || NL == 2 || NL == 4 || NL == 8), "stats_ls shape");
    __shared__ __align__(16) char lds[NL * LEAF_BYTES];
    __shared__ float lmax[NL][2][4];
    // fp32 rows: per wave 2 KB to turn 4 centres' rows into whole-row stores (below)
    __shared__ __align__(16) char rowbuf[STORE == 3 ? 4 : 1][STORE == 3 ? 2048 : 16];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // 1-D grid over (centre part, leaf group, head), centre part fastest: the workgroups of one
    // head run together on one XCD, whose L2 then serves the head's centres to all of them
    const int nlg = nb_pad / NL;
    const uint32_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int cs = (int)(blk % (uint32_t)ncs), lg = (int)((blk / (uint32_t)ncs) % (uint32_t)nlg);
    const int h = (int)(blk / ((uint32_t)ncs * (uint32_t)nlg));
    const int l0 = lg * NL;
    const int lr = min(nb, l0 + NL);              // real leaves [l0, lr)
    const int64_t kh = (int64_t)h * nk;
    const int ncg = (nt + 15) / 16, gpp = (ncg + ncs - 1) / ncs;
    const int jb = cs * gpp, je = min(ncg, jb + gpp);
    const float sl2 = __fmul_rn(scale, LOG2E);
    int tk[NL], tv[NL];
    stage_leaves_f16<LEAF, NL>(k, v, kh + (int64_t)l0 * LEAF, lr - l0, lds, lmax, tk, tv);
    // this lane's 32 centre values (dims 32 ks + 8 grp + e of centre 16 j + col), fp32; with
    // precomputed terms (mut, centre_terms_kernel) their hi / lo fp16 words in the same registers
    // (m[2 ks] hi, m[2 ks + 1] lo) and the centre's exponent in sm
    auto load_mu = [&](int j, f32x4 (&m)[8], int& sm) {
        const int t = min(16 * j + col, nt - 1);
        if constexpr (MUT) {
            const uint16_t* src = mut + ((int64_t)h * nt + t) * MUT_ROW + 8 * grp;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                m[2 * ks] = *(const f32x4*)(src + 32 * ks);
                m[2 * ks + 1] = *(const f32x4*)(src + D + 32 * ks);
            }
            sm = *(const int*)(mut + ((int64_t)h * nt + t) * MUT_ROW + 2 * D);
            return;
        }
        const float* src = mu + ((int64_t)h * mu_stride + c0 + t) * D + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            m[2 * ks] = *(const f32x4*)(src + 32 * ks);
            m[2 * ks + 1] = *(const f32x4*)(src + 32 * ks + 4);
        }
    };
    // mu of a group scaled by 2^smu (per centre: its largest |value| into [2^14, 2^15), smu in
    // [-64, 64]) and split into two fp16 terms (the logits, and through the softmax g, carry no
    // error beyond fp32 rounding)
    u32x4 mh[4], ml[4];
    int smu = 0;
    auto split_mu = [&](const f32x4 (&m)[8], int sm) {
        if constexpr (MUT) {
            smu = sm;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                mh[ks] = __builtin_bit_cast(u32x4, m[2 * ks]);
                ml[ks] = __builtin_bit_cast(u32x4, m[2 * ks + 1]);
            }
            return;
        }
        float mx = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(m[q][e]));
        mx = grp_max(mx);
        const int e = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 127;
        smu = 14 - e < -64 ? -64 : (14 - e > 64 ? 64 : 14 - e);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float x[8];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {    // (TF32: the operand rounded first; lo is then 0)
                x[e2] = ldexpf(TF32 ? tf32_rna(m[2 * ks][e2]) : m[2 * ks][e2], smu);
                x[4 + e2] = ldexpf(TF32 ? tf32_rna(m[2 * ks + 1][e2]) : m[2 * ks + 1][e2], smu);
            }
            split2h8(x, mh[ks], ml[ks]);
        }
    };
    f32x4 mnext[8];
    int snext = 0;
    if (jb + w < je) {
        load_mu(jb + w, mnext, snext);
        split_mu(mnext, snext);
    }
    for (int j = jb + w; j < je; j += 4) {
        // Centres past the last (t >= nt) compute and store the last centre's state: the same bits
        // to the same rows.  Every store is unconditional and the next group's centres are loaded
        // at the top of the iteration (a valid group even past the wave's last) and split at its
        // end, so the compiler's wait for them counts the iteration's stores issued after them
        // instead of draining them all.
        const int64_t th = (int64_t)h * nt + min(16 * j + col, nt - 1);
        load_mu(min(j + 4, je - 1), mnext, snext);
        float sgs[NL], lzs[NL], svs[NL];
#pragma unroll
        for (int li = 0; li < NL; ++li) {
            sgs[li] = 0.0f;
            lzs[li] = -INFINITY;
            svs[li] = 0.0f;
        }
        // padded leaf: empty state, excluded everywhere (zero rows by the store instructions of a
        // real leaf: the same count on both paths)
        auto pad_leaf = [&](int li) {
            const int64_t s = th * nb_pad + l0 + li;
            if (F32) {
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    *(u32x4*)((float*)g8 + s * D + 16 * db + 4 * grp) = u32x4{0u, 0u, 0u, 0u};
                    *(u32x4*)((float*)vb + s * D + 16 * db + 4 * grp) = u32x4{0u, 0u, 0u, 0u};
                }
                return;
            }
            if (BF16) {
                *(u32x4*)((uint16_t*)g8 + s * D + 8 * grp) = u32x4{0u, 0u, 0u, 0u};
                *(u32x4*)((uint16_t*)g8 + s * D + 32 + 8 * grp) = u32x4{0u, 0u, 0u, 0u};
                *(u32x4*)((uint16_t*)g8 + s * D + 64 + 8 * grp) = u32x4{0u, 0u, 0u, 0u};
                *(u32x4*)((uint16_t*)g8 + s * D + 96 + 8 * grp) = u32x4{0u, 0u, 0u, 0u};
            } else {
                *(u32x4*)(g8 + s * D + 16 * grp) = u32x4{0u, 0u, 0u, 0u};
                *(u32x4*)(g8 + s * D + 64 + 16 * grp) = u32x4{0u, 0u, 0u, 0u};
            }
            if (FP8) {
                *(u32x4*)((uint8_t*)vb + s * D + 16 * grp) = u32x4{0u, 0u, 0u, 0u};
                *(u32x4*)((uint8_t*)vb + s * D + 64 + 16 * grp) = u32x4{0u, 0u, 0u, 0u};
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) *(u32x4*)(vb + s * D + 32 * q + 8 * grp) = u32x4{0u, 0u, 0u, 0u};
            }
        };
        auto real_leaf = [&](int li) {
            const int64_t s = th * nb_pad + l0 + li;
            const char* Kr = lds + li * LEAF_BYTES;
            const char* Vr = Kr + 16 * LEAF * 16;
            // a' = a 2^(smu - tk): the logits' power of two ca = tk - smu goes into their scale
            const int ca = tk[li] - smu;
            const float sca = ldexpf(scale, ca), sl2a = ldexpf(sl2, ca);
            // QK by k-steps ks: the K operands of the KB key blocks for step ks + 1 are read from
            // LDS while step ks's products run, and each step's products alternate over the KB
            // accumulators (lo terms, then hi terms) so no product waits on the one before it
            auto qk_op = [&](int kb, int ks) {
                const int row = 16 * kb + col;
                return *(const u32x4*)(Kr + (row * 16 + ((4 * ks + grp) ^ swz(row))) * 16);
            };
            f32x4 a[KB];
            u32x4 aop[2][KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                a[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                aop[0][kb] = qk_op(kb, 0);
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks + 1 < 4) {
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) aop[(ks + 1) & 1][kb] = qk_op(kb, ks + 1);
                }
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)                  // smaller term first
                    if constexpr (!TF32) a[kb] = mfma_f16(aop[ks & 1][kb], ml[ks], a[kb]);
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) a[kb] = mfma_f16(aop[ks & 1][kb], mh[ks], a[kb]);
            }
            float amx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) amx = fmaxf(amx, a[kb][i]);
            amx = grp_max(amx);
            const float mx = __fmul_rn(amx, sca), mlog = __fmul_rn(amx, sl2a);
            float z = 0.0f;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a[kb][i] = __builtin_amdgcn_exp2f(__fmaf_rn(a[kb][i], sl2a, -mlog));
                    z = __fadd_rn(z, a[kb][i]);
                }
            z = grp_sum(z);
            // w 2^14 (in [0, 2^14]): the weights' low fp16 terms stay normal down to w = 2^-14
            const float rz = __fmul_rn(__fdiv_rn(1.0f, z), 16384.0f);
            f32x4 gacc[8], vacc[8];
#pragma unroll
            for (int db = 0; db < 8; ++db) gacc[db] = vacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
            u32x4 W1[KK], W0[KK];
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                float wv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int kb = 2 * kk + (e >> 2);
                    wv[e] = kb < KB ? __fmul_rn(a[kb < KB ? kb : 0][e & 3], rz) : 0.0f;
                    if constexpr (TF32) wv[e] = tf32_rna(wv[e]);
                }
                split2h8(wv, W1[kk], W0[kk]);
            }
            // PV over steps p = (kk, db): each step's K^T / V^T operands are read from LDS one
            // step ahead of its four products
            constexpr int NP = 8 * KK;
            auto pv_op = [&](int p, u32x4& ka, u32x4& va) {
                const int kk = p / 8, db = p % 8;
                const u32x2 zero = {0u, 0u};
                const u32x2 k0 = tr_operand(Kr, 32 * kk, db, lane);
                const u32x2 k1 = (2 * kk + 1 < KB) ? tr_operand(Kr, 32 * kk + 16, db, lane) : zero;
                const u32x2 v0 = tr_operand(Vr, 32 * kk, db, lane);
                const u32x2 v1 = (2 * kk + 1 < KB) ? tr_operand(Vr, 32 * kk + 16, db, lane) : zero;
                ka = u32x4{k0.x, k0.y, k1.x, k1.y};
                va = u32x4{v0.x, v0.y, v1.x, v1.y};
            };
            u32x4 kop[2], vop[2];
            pv_op(0, kop[0], vop[0]);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int kk = p / 8, db = p % 8;
                const u32x4 KA = kop[p & 1], VA = vop[p & 1];
                if (p + 1 < NP) pv_op(p + 1, kop[(p + 1) & 1], vop[(p + 1) & 1]);
                if constexpr (!TF32) gacc[db] = mfma_f16(KA, W0[kk], gacc[db]);
                gacc[db] = mfma_f16(KA, W1[kk], gacc[db]);
                if constexpr (!TF32) vacc[db] = mfma_f16(VA, W0[kk], vacc[db]);
                vacc[db] = mfma_f16(VA, W1[kk], vacc[db]);
            }
            lzs[li] = __fadd_rn(mx, ln_ge1(z));   // z >= 1: its largest term is exp(0)
            // gacc = g 2^(14 - tk) / scale, vacc = vb 2^(14 - tv)
            const float scg = ldexpf(scale, tk[li] - 14);
            const int ev = tv[li] - 14;
            // vb = vacc 2^ev by one multiply (ev in [-38, 100]: 2^ev is a normal float, and the
            // rounded product is the ldexp result; v_mul_f32 issues at about 1.6x v_ldexp_f32's rate)
            const float pev = ldexpf(1.0f, ev);
            float am = 0.0f;
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) am = fmaxf(am, fabsf(gacc[db][i]));
            am = __fmul_rn(grp_max(am), scg);     // max |g|
            // one-byte rows (g8, FP8 g / vb): 4 x 4 block transpose of (c[g], c[4 + g]); row g then
            // holds dims 16g + 4c in x[2c] and 64 + 16g + 4c in x[2c + 1]: each store instruction
            // writes 64 contiguous bytes of a row per lane group
            auto store_bytes = [&](const uint32_t (&c)[8], uint8_t* dst) {
                uint32_t x[8] = {c[0], c[4], c[1], c[5], c[2], c[6], c[3], c[7]};
                rows_transpose(x);
                *(u32x4*)(dst + s * D + 16 * grp) = u32x4{x[0], x[2], x[4], x[6]};
                *(u32x4*)(dst + s * D + 64 + 16 * grp) = u32x4{x[1], x[3], x[5], x[7]};
            };
            // bf16 rows, both halves hf (dims 64 hf ..): rows 2j and 2j + 1 swap halves; row g then
            // holds, for db = 2m + (g & 1), dims 16db + 8(g >> 1) .. + 3 in va and .. + 4 .. + 7 in vc
            auto store_rows16 = [&](const u32x2 (&c)[8], uint16_t* dst) {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    u32x2 va[2], vc[2];
#pragma unroll
                    for (int m2 = 0; m2 < 2; ++m2) {
                        const int m = 2 * hf + m2;
                        uint32_t a0 = c[2 * m].x, a1 = c[2 * m].y, cc0 = c[2 * m + 1].x, cc1 = c[2 * m + 1].y;
                        swap16(a0, cc0);
                        swap16(a1, cc1);
                        va[m2] = u32x2{a0, a1};
                        vc[m2] = u32x2{cc0, cc1};
                    }
                    uint16_t* vr = dst + s * D + 16 * (grp & 1) + 8 * (grp >> 1);
#pragma unroll
                    for (int m2 = 0; m2 < 2; ++m2)
                        *(u32x4*)(vr + 32 * (2 * hf + m2)) = u32x4{va[m2].x, va[m2].y, vc[m2].x, vc[m2].y};
                }
            };
            if constexpr (F32) {
                // fp32 rows (the lane holds dims 16 db + 4 grp .. of centre col) through this wave's
                // 2 KB of LDS, 4 centres at a time, so each store instruction writes two whole
                // 512-byte rows instead of 16 rows' 64-byte pieces (cfg3: 7.13 -> 5.3 ms when every
                // store instruction is one contiguous KB).  Buffered row rr keeps its 16-byte chunk c
                // (dims 4 c ..) at c ^ 4 rr: the 16 writing lanes and the 32 lanes reading a row
                // address distinct banks.
                char* tb = &rowbuf[w][0];
                const int hl = lane >> 5, cl = lane & 31;
                auto put = [&](const f32x4 (&acc)[8], float sc, float* dst) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if ((col >> 2) == r) {
                            const int rr = col & 3;
#pragma unroll
                            for (int db = 0; db < 8; ++db)
                                *(f32x4*)(tb + rr * 512 + (((4 * db + grp) ^ (4 * rr)) << 4)) =
                                    f32x4{__fmul_rn(acc[db][0], sc), __fmul_rn(acc[db][1], sc),
                                          __fmul_rn(acc[db][2], sc), __fmul_rn(acc[db][3], sc)};
                        }
                        wave_lds_sync();               // the 4 rows written before any lane reads them
#pragma unroll
                        for (int ii = 0; ii < 2; ++ii) {
                            const int rr = 2 * ii + hl, cc = 4 * r + rr;
                            const f32x4 v4 = *(const f32x4*)(tb + rr * 512 + ((cl ^ (4 * rr)) << 4));
                            const int64_t sr = ((int64_t)h * nt + min(16 * j + cc, nt - 1)) * nb_pad + l0 + li;
                            *(f32x4*)(dst + sr * D + 4 * cl) = v4;
                        }
                        wave_lds_sync();               // read before the next 4 rows overwrite them
                    }
                };
                put(gacc, scg, (float*)g8);
                put(vacc, pev, (float*)vb);
            } else if constexpr (BF16) {
                u32x2 pgb[8], pv[8];
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    pgb[db] = u32x2{pack2bf(__fmul_rn(gacc[db][0], scg), __fmul_rn(gacc[db][1], scg)),
                                    pack2bf(__fmul_rn(gacc[db][2], scg), __fmul_rn(gacc[db][3], scg))};
                    pv[db] = u32x2{pack2bf(__fmul_rn(vacc[db][0], pev), __fmul_rn(vacc[db][1], pev)),
                                   pack2bf(__fmul_rn(vacc[db][2], pev), __fmul_rn(vacc[db][3], pev))};
                }
                store_rows16(pgb, (uint16_t*)g8);
                store_rows16(pv, vb);
            } else if constexpr (FP8) {
                const float sgv = fmaxf(__fmul_rn(am, R448), 1e-30f);
                float av = 0.0f;
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int i = 0; i < 4; ++i) av = fmaxf(av, fabsf(vacc[db][i]));
                const float svv = fmaxf(__fmul_rn(ldexpf(grp_max(av), ev), R448), 1e-30f);
                const float cg = __fdiv_rn(scg, sgv), cv = ldexpf(__fdiv_rn(1.0f, svv), ev);
                uint32_t pg[8], pvc[8];
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    pg[db] = quant4_e4m3_cvt(gacc[db], cg);
                    pvc[db] = quant4_e4m3_cvt(vacc[db], cv);
                }
                store_bytes(pg, (uint8_t*)g8);
                store_bytes(pvc, (uint8_t*)vb);
                sgs[li] = sgv;
                svs[li] = svv;
            } else {
                am = am < 1e-30f ? 1e-30f : am;
                const float cq = __fdiv_rn(__fmul_rn(127.0f, scg), am);
                uint32_t pg[8];
                u32x2 pv[8];
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    pg[db] = quant4(gacc[db], cq);
                    pv[db] = u32x2{pack2bf(__fmul_rn(vacc[db][0], pev), __fmul_rn(vacc[db][1], pev)),
                                   pack2bf(__fmul_rn(vacc[db][2], pev), __fmul_rn(vacc[db][3], pev))};
                }
                store_bytes(pg, (uint8_t*)g8);
                store_rows16(pv, vb);
                sgs[li] = __fmul_rn(am, R127);
            }
        };
        if (lr - l0 == NL) {                        // every leaf real: one straight-line body
#pragma unroll
            for (int li = 0; li < NL; ++li) real_leaf(li);
        } else {
#pragma unroll
            for (int li = 0; li < NL; ++li) {
                if (l0 + li >= lr) pad_leaf(li);
                else real_leaf(li);
            }
        }
        // sg, lz (sv) of the NL leaves: NL contiguous floats per centre (the four lanes of a column
        // hold the same values and write them alike)
        {
            const int64_t s = th * nb_pad + l0;
            auto put = [&](float* dst, const float (&x)[NL]) {
                if constexpr (NL == 1) {
                    dst[s] = x[0];
                } else if constexpr (NL == 2) {
                    *(u32x2*)(dst + s) = u32x2{__float_as_uint(x[0]), __float_as_uint(x[1])};
                } else {
#pragma unroll
                    for (int q = 0; q < NL; q += 4) *(f32x4*)(dst + s + q) = f32x4{x[q], x[q + 1], x[q + 2], x[q + 3]};
                }
            };
            if (HAS_SG) put(sg, sgs);
            put(lz, lzs);
            if (FP8) put(sv, svs);
        }
        split_mu(mnext, snext);
    }
}

// ---------------------------------------------------------------------------------------------
// select: SEL[t, l] = max_r float(dq8_r . g8_tl) * (sdq_r * sg_tl) + lz_tl
// (h3/htrc_flat_triton.py:214-254).  Workgroup = one tile x 256 leaves; each wave owns 64
// leaves and all rows (tile / 16 B operands of 16 rows held in registers).  Bit-exact: int32 dot,
// one fp32 product per row, an exact max, one fp32 add.
// ---------------------------------------------------------------------------------------------
template <int NRB>
__device__ __forceinline__ void load_rows_i8(const int8_t* __restrict__ x8, int64_t row0, int stride,
                                             int ts, int col, int grp, i32x4 (&b)[NRB][2], bool (&val)[NRB]) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
        const int r = 16 * rb + col;
        val[rb] = r < ts;
        const int64_t p = row0 + (int64_t)(val[rb] ? r : 0) * stride;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) b[rb][ks] = *(const i32x4*)(x8 + p * D + 64 * ks + 16 * grp);
    }
}

// SEL of one tile group (G tiles sharing a centre; G = 1: one tile): the max runs over the
// rows of every tile of the group (h3/htrc_flat.py:244-252 hands the kernel the G * tile rows).
// NRB = tile / 16 row blocks of 16 rows held as B operands.
template <int NRB>
__global__ __launch_bounds__(256) void select_kernel(const int8_t* __restrict__ dq8,
                                                     const float* __restrict__ sdq, int stride,
                                                     const int8_t* __restrict__ g8,
                                                     const float* __restrict__ sg,
                                                     const float* __restrict__ lz, int nt, int group, int g0,
                                                     int ng, int nb, int nb_pad, float* __restrict__ sel) {
    constexpr int TR = 16 * NRB;                      // rows per tile
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int gi = blockIdx.x, h = blockIdx.z;
    const int64_t gs = (int64_t)h * ng + gi;          // state / SEL row of the group (the launch's window)
    const int ts = TR / stride;
    const int c0 = blockIdx.y * 256 + w * 64;
    float bsel[4][4];
#pragma unroll
    for (int lb = 0; lb < 4; ++lb)
#pragma unroll
        for (int i = 0; i < 4; ++i) bsel[lb][i] = -INFINITY;
    for (int j = 0; j < group; ++j) {
        const int t = (g0 + gi) * group + j;
        if (t >= nt) break;                           // padded tiles repeat the last one
        const int64_t th = (int64_t)h * nt + t;
        i32x4 b[NRB][2];
        bool val[NRB];
        load_rows_i8(dq8, th * TR, stride, ts, col, grp, b, val);
        float srow[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) srow[rb] = sdq[th * TR + (int64_t)(val[rb] ? 16 * rb + col : 0) * stride];
#pragma unroll
        for (int lb = 0; lb < 4; ++lb) {
            const int c = c0 + 16 * lb;
            if (c < nb) {
                const int64_t s0 = gs * nb_pad + c;
                const int8_t* G = g8 + s0 * D;
                i32x4 acc[NRB];
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) acc[rb] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const i32x4 A = *(const i32x4*)(G + col * D + 64 * ks + 16 * grp);
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb) acc[rb] = mfma_i8(A, b[rb][ks], acc[rb]);
                }
                const f32x4 sgv = *(const f32x4*)(sg + s0 + 4 * grp);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float best = -INFINITY;
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
                        best = fmaxf(best, __fmul_rn((float)acc[rb][i], __fmul_rn(srow[rb], sgv[i])));   // rows past ts repeat row 0
                    bsel[lb][i] = fmaxf(bsel[lb][i], col_max(best));
                }
            }
        }
    }
    if (col == 0) {
#pragma unroll
        for (int lb = 0; lb < 4; ++lb) {
            const int c = c0 + 16 * lb;
            if (c >= nb) break;
            const f32x4 lzv = *(const f32x4*)(lz + gs * nb_pad + c + 4 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int l = c + 4 * grp + i;
                if (l < nb) sel[gs * nb_pad + l] = __fadd_rn(bsel[lb][i], lzv[i]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Top-k of one SEL row by 8-bit MSB-first radix select in LDS, then an ascending-index
// compaction (ties at the threshold go to the lower leaf index).  Leaves < sink are
// forced in (h3/htrc_flat.py:262-265).  Used by the topk kernel and the fused route kernel.
// ---------------------------------------------------------------------------------------------
struct TopkSmem {
    uint32_t hist[256];
    uint32_t cnt_gt[257];
    uint32_t cnt_eq[257];
    uint32_t prefix, remaining;
};

// Small kx (<= 64), idx only: the same set as the radix select below, from a lower bound of the
// threshold.  Wave 0 takes the maxima of the 64 strided subsets l = j (mod 64) and sorts them
// (bitonic, across the lanes); the kx-th largest, L, has kx subsets holding a key >= L, so at
// least kx keys are >= L and the kx-th largest key is too.  The keys >= L (a few more than kx
// for score rows) are compacted in leaf order and each is ranked exactly: keys above it, and
// equal keys at lower leaves.  More than 256 candidates (many equal keys): returns false before
// anything is written, and the radix select runs.  Five barriers, every thread through each.
template <typename Keys>
__device__ bool topk_small(Keys keys, int nb, int kx, TopkSmem& sm, int32_t* idx_out) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t* ck = sm.hist;        // candidate keys
    uint32_t* cl = sm.cnt_gt;      // candidate leaves
    if (wv == 0) {
        uint32_t m = 0;            // below every order key of a real score
#pragma unroll 4
        for (int l = lane; l < nb; l += 64) m = max(m, keys(l));
#pragma unroll
        for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {   // blocks of k descending where lane & k == 0
                const uint32_t o = (uint32_t)__shfl_xor((int)m, j, 64);
                m = (((lane & j) == 0) == ((lane & k) == 0)) ? max(m, o) : min(m, o);
            }
        if (lane == kx - 1) sm.prefix = m;
    }
    __syncthreads();
    const uint32_t lb = sm.prefix;
    const int chunk = (nb + 255) / 256;
    const int a = min(nb, tid * chunk), b = min(nb, a + chunk);
    uint32_t n = 0;
    for (int l = a; l < b; ++l) n += keys(l) >= lb;
    uint32_t incl = n;             // inclusive prefix over the wave, then the waves before
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) sm.cnt_eq[wv] = incl;
    __syncthreads();
    uint32_t off = incl - n, nc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = sm.cnt_eq[j];
        if (j < wv) off += c;
        nc += c;
    }
    if (nc > 256) return false;    // the same nc in every thread
    for (int l = a; l < b; ++l) {
        const uint32_t key = keys(l);
        if (key >= lb) {
            ck[off] = key;
            cl[off] = (uint32_t)l;
            ++off;
        }
    }
    __syncthreads();
    bool sel = false;
    uint32_t leaf = 0;
    if ((uint32_t)tid < nc) {
        const uint32_t key = ck[tid];
        uint32_t r = 0;
#pragma unroll 8
        for (uint32_t j = 0; j < nc; ++j) {
            const uint32_t kj = ck[j];
            r += (kj > key || (kj == key && j < (uint32_t)tid)) ? 1u : 0u;
        }
        sel = r < (uint32_t)kx;
        leaf = cl[tid];
    }
    const uint64_t bal = __ballot(sel);   // output position: selected candidates before this one
    if (lane == 0) sm.cnt_eq[4 + wv] = (uint32_t)__popcll(bal);
    __syncthreads();
    uint32_t pos = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
    for (int j = 0; j < wv; ++j) pos += sm.cnt_eq[4 + j];
    if (sel) idx_out[pos] = (int32_t)leaf;
    __syncthreads();
    return true;
}

// keys(l) is order_key(sel[l]) for l < nb (an LDS array, or computed from global memory for rows
// longer than the LDS holds).  Writes idx[0..kx) ascending and (optionally) excl.
template <typename Keys>
__device__ void topk_row(Keys keys, int nb, int kx, TopkSmem& sm, int32_t* idx_out,
                         int8_t* excl_out, int32_t* idx_lds) {
    const int tid = threadIdx.x;
    if (kx >= nb) {               // everything is selected
        for (int l = tid; l < nb; l += 256) {
            if (idx_out) idx_out[l] = l;
            if (idx_lds) idx_lds[l] = l;
            if (excl_out) excl_out[l] = 1;
        }
        __syncthreads();
        return;
    }
    if (kx <= 64 && idx_out && !excl_out && !idx_lds && topk_small(keys, nb, kx, sm, idx_out)) return;
    if (tid == 0) {
        sm.prefix = 0;
        sm.remaining = (uint32_t)kx;
    }
    uint32_t mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sm.hist[tid] = 0;
        __syncthreads();
        const uint32_t prefix = sm.prefix;
        for (int l = tid; l < nb; l += 256) {
            const uint32_t key = keys(l);
            if ((key & mask) == prefix) atomicAdd(&sm.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {            // one wave: find the digit where the count from the top reaches `remaining`
            const int lane = tid;
            uint32_t c[4], s = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {          // lane owns digits 255-4*lane .. 252-4*lane
                c[j] = sm.hist[255 - (4 * lane + j)];
                s += c[j];
            }
            uint32_t incl = s;                     // inclusive prefix over lanes (descending digits)
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_up(incl, o, 64);
                if (lane >= o) incl += y;
            }
            const uint32_t excl_before = incl - s;
            const uint32_t rem = sm.remaining;
            uint32_t run = excl_before;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (run < rem && run + c[j] >= rem) {
                    const uint32_t digit = 255u - (uint32_t)(4 * lane + j);
                    sm.prefix = prefix | (digit << shift);
                    sm.remaining = rem - run;
                }
                run += c[j];
            }
        }
        mask |= 255u << shift;
        __syncthreads();
    }
    const uint32_t thr = sm.prefix, need_eq = sm.remaining;
    // ascending compaction: thread owns a contiguous chunk of leaves
    const int chunk = (nb + 255) / 256;
    const int a = min(nb, tid * chunk), b = min(nb, a + chunk);
    uint32_t ngt = 0, neq = 0;
    for (int l = a; l < b; ++l) {
        const uint32_t key = keys(l);
        ngt += key > thr;
        neq += key == thr;
    }
    {   // exclusive prefix over the 256 threads: in-wave inclusive scan, then wave offsets
        const int lane = tid & 63, wv = tid >> 6;
        uint32_t ig = ngt, ie = neq;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t yg = __shfl_up(ig, o, 64), ye = __shfl_up(ie, o, 64);
            if (lane >= o) {
                ig += yg;
                ie += ye;
            }
        }
        if (lane == 63) {
            sm.cnt_gt[wv] = ig;
            sm.cnt_eq[wv] = ie;
        }
        __syncthreads();
        uint32_t og = 0, oe = 0;
        for (int j = 0; j < wv; ++j) {
            og += sm.cnt_gt[j];
            oe += sm.cnt_eq[j];
        }
        __syncthreads();
        sm.cnt_gt[tid] = og + ig - ngt;
        sm.cnt_eq[tid] = oe + ie - neq;
        __syncthreads();
    }
    uint32_t eqr = sm.cnt_eq[tid];
    uint32_t pos = sm.cnt_gt[tid] + (eqr < need_eq ? eqr : need_eq);
    for (int l = a; l < b; ++l) {
        const uint32_t key = keys(l);
        bool take = key > thr;
        if (key == thr) {
            take = eqr < need_eq;
            ++eqr;
        }
        take = take && pos < (uint32_t)kx;   // never more than kx, whatever the counts say
        if (excl_out) excl_out[l] = take ? 1 : 0;
        if (take) {
            if (idx_out) idx_out[pos] = l;
            if (idx_lds) idx_lds[pos] = l;
            ++pos;
        }
    }
    __syncthreads();
}

constexpr int MAX_NB_LDS = 8192;   // leaves per head the LDS top-k keys hold (longer rows: global)

// One workgroup per SEL row.  LDS_KEYS: the row's keys staged in LDS; otherwise each radix pass
// reads the row from global memory (L2) and forms the keys on the fly.
template <bool LDS_KEYS>
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ sel, int nb, int nb_pad,
                                                   int kx, int sink, int32_t* __restrict__ idx,
                                                   int8_t* __restrict__ excl) {
    __shared__ uint32_t keys[LDS_KEYS ? MAX_NB_LDS : 1];
    __shared__ TopkSmem sm;
    const int64_t row = blockIdx.x;
    const float* srow = sel + row * nb_pad;
    for (int l = nb + threadIdx.x; l < nb_pad; l += 256) excl[row * nb_pad + l] = 0;
    if constexpr (LDS_KEYS) {
        for (int l = threadIdx.x; l < nb; l += 256) keys[l] = l < sink ? 0xffffffffu : order_key(srow[l]);
        __syncthreads();
        topk_row([&](int l) { return keys[l]; }, nb, kx, sm, idx + row * kx, excl + row * nb_pad, nullptr);
    } else {
        topk_row([&](int l) { return l < sink ? 0xffffffffu : order_key(srow[l]); }, nb, kx, sm, idx + row * kx,
                 excl + row * nb_pad, nullptr);
    }
}

// ---------------------------------------------------------------------------------------------
// tile: far field + near field online softmax for one (tile, split)
// (h3/htrc_flat_triton.py:88-211, DOT=1, I8=1).  Four waves x 16 query rows.  Far leaves in
// blocks of 32: S^T = g8 dq8^T (int8 MFMA), p = exp(score - m), O^T += vb^T p^T (bf16 MFMA).
// Near tokens in blocks of 32 (two 16-key runs of selected leaves): S^T = k8 q8^T,
// O^T += v^T p^T.  O^T keeps the query row on lane%16, so rescaling needs no shuffles.
// ---------------------------------------------------------------------------------------------
struct RowState {
    float m;     // running max (same in the four lanes of a row)
    float l;     // this lane's share of the running sum
    f32x4 o[8];  // O^T: dims 16db + 4grp + i of row lane%16
};

// Online update with the scores of this lane's 8 keys (sc[0..7]) and the PV operand
// fetch functor for the 8 dim-blocks.
template <typename VFetch>
__device__ __forceinline__ void online_block(RowState& st, float (&sc)[8], VFetch&& vfetch) {
    float bm = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) bm = fmaxf(bm, sc[e]);
    bm = grp_max(bm);
    const float m_new = fmaxf(st.m, bm);
    const float m_s = m_new == -INFINITY ? 0.0f : m_new;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = __expf(__fsub_rn(sc[e], m_s));
        ps = __fadd_rn(ps, p[e]);
    }
    const float alpha = __expf(__fsub_rn(st.m, m_s));
    st.l = __fadd_rn(__fmul_rn(st.l, alpha), ps);
    const bf16x8 P = to_bf16x8(p);
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        f32x4 o = st.o[db];
        o[0] = __fmul_rn(o[0], alpha);
        o[1] = __fmul_rn(o[1], alpha);
        o[2] = __fmul_rn(o[2], alpha);
        o[3] = __fmul_rn(o[3], alpha);
        st.o[db] = mfma_bf16(vfetch(db), P, o);
    }
    st.m = m_new;
}

// PV operand from a natural-layout bf16 matrix X[row][128]: rows r0 + 4grp + i and
// r1 + 4grp + i (i = 0..3) at column dim.
__device__ __forceinline__ bf16x8 gather_pv(const uint16_t* __restrict__ X, int64_t r0, int64_t r1, int dim, int grp) {
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint16_t* b = X + ((j ? r1 : r0) + 4 * grp) * D + dim;
        u[2 * j] = (uint32_t)b[0] | ((uint32_t)b[D] << 16);
        u[2 * j + 1] = (uint32_t)b[2 * D] | ((uint32_t)b[3 * D] << 16);
    }
    return as_bf16x8(u32x4{u[0], u[1], u[2], u[3]});
}

template <int LEAF>
__device__ __forceinline__ void tile_far_near(RowState& st, int64_t srow, int nb, int nb_pad,
                                              int lo, int hi, int e_lo, int e_hi, int kx,
                                              const i32x4 (&q8r)[2], float sqr, const i32x4 (&dq8r)[2],
                                              float sdqr, const int8_t* __restrict__ g8,
                                              const float* __restrict__ sg, const float* __restrict__ lz,
                                              const uint16_t* __restrict__ vb,
                                              const int8_t* __restrict__ excl_row,
                                              const int32_t* __restrict__ idx_row,
                                              const int8_t* __restrict__ k8,
                                              const float* __restrict__ ks,
                                              const uint16_t* __restrict__ v, int64_t kh, float scale) {
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // ---- far field
    for (int c0 = lo; c0 < hi; c0 += 32) {
        float sc[8];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int cb = c0 + 16 * h2;
            const int64_t s0 = srow * nb_pad + cb;
            i32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kss = 0; kss < 2; ++kss) {
                const i32x4 A = *(const i32x4*)(g8 + (s0 + col) * D + 64 * kss + 16 * grp);
                acc = mfma_i8(A, dq8r[kss], acc);
            }
            const f32x4 sgv = *(const f32x4*)(sg + s0 + 4 * grp);
            const f32x4 lzv = *(const f32x4*)(lz + s0 + 4 * grp);
            const uint32_t exv = *(const uint32_t*)(excl_row + cb + 4 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = cb + 4 * grp + i;
                const bool ok = c < hi && ((exv >> (8 * i)) & 0xffu) == 0u;
                sc[4 * h2 + i] = ok ? __fadd_rn(__fmul_rn((float)acc[i], __fmul_rn(sdqr, sgv[i])), lzv[i]) : -INFINITY;
            }
        }
        const uint16_t* vb0 = vb + (srow * nb_pad + c0) * D;
        online_block(st, sc, [&](int db) { return gather_pv(vb0, 0, 16, 16 * db + col, grp); });
    }
    // ---- near field: token j of the tile's selected list -> idx[j / LEAF] * LEAF + j % LEAF
    for (int e0 = e_lo; e0 < e_hi; e0 += 32) {
        float sc[8];
        int64_t tok0[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int j0 = e0 + 16 * h2;
            const bool ok = j0 < e_hi;
            const int jj = ok ? j0 : e_lo;
            tok0[h2] = kh + (int64_t)idx_row[jj / LEAF] * LEAF + (jj % LEAF);
            i32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kss = 0; kss < 2; ++kss) {
                const i32x4 A = *(const i32x4*)(k8 + (tok0[h2] + col) * D + 64 * kss + 16 * grp);
                acc = mfma_i8(A, q8r[kss], acc);
            }
            const f32x4 ksv = *(const f32x4*)(ks + tok0[h2] + 4 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool oki = ok && (j0 + 4 * grp + i) < e_hi;
                sc[4 * h2 + i] = oki ? __fmul_rn((float)acc[i], __fmul_rn(__fmul_rn(sqr, ksv[i]), scale)) : -INFINITY;
            }
        }
        online_block(st, sc, [&](int db) { return gather_pv(v, tok0[0], tok0[1], 16 * db + col, grp); });
    }
}

__device__ __forceinline__ void load_row_ops(const int8_t* __restrict__ q8, const int8_t* __restrict__ dq8,
                                             int64_t p, int grp, i32x4 (&q8r)[2], i32x4 (&dq8r)[2]) {
#pragma unroll
    for (int kss = 0; kss < 2; ++kss) {
        q8r[kss] = *(const i32x4*)(q8 + p * D + 64 * kss + 16 * grp);
        dq8r[kss] = *(const i32x4*)(dq8 + p * D + 64 * kss + 16 * grp);
    }
}

// Final normalisation of a row state (one split): out = O / max(l, 1e-30), logZ = m_s + log l.
__device__ __forceinline__ void write_final(const RowState& st, float ltot, int64_t orow, bool valid,
                                            float* __restrict__ out, float* __restrict__ logz) {
    const int lane = threadIdx.x & 63, grp = lane >> 4;
    if (!valid) return;
    const float ms = st.m == -INFINITY ? 0.0f : st.m;
    const float den = ltot < 1e-30f ? 1e-30f : ltot;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = __fdiv_rn(st.o[db][i], den);
        *(f32x4*)(out + orow * D + 16 * db + 4 * grp) = o;
    }
    if (grp == 0) logz[orow] = __fadd_rn(ms, __logf(ltot));
}

template <int LEAF>
__global__ __launch_bounds__(256) void tile_kernel(
    const int8_t* __restrict__ q8, const float* __restrict__ sq, const int8_t* __restrict__ dq8,
    const float* __restrict__ sdq, const int8_t* __restrict__ g8, const float* __restrict__ sg,
    const float* __restrict__ lz, const uint16_t* __restrict__ vb, const int8_t* __restrict__ excl,
    const int32_t* __restrict__ idx, const int8_t* __restrict__ k8, const float* __restrict__ ks,
    const uint16_t* __restrict__ v, int64_t nq, int nt, int tile, int group, int g0, int ng,
    const int32_t* __restrict__ perm, int64_t nk, int nb, int nb_pad, int kx, int lps, int eps, float scale,
    float* __restrict__ pm, float* __restrict__ pl, float* __restrict__ pacc,
    float* __restrict__ out, float* __restrict__ logz) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // tiles of groups [g0, g0 + ng): state, routing and partial rows are the launch's own
    const int tb = g0 * group, ntw = gridDim.x;
    const int t = tb + blockIdx.x, sp = blockIdx.y, ns = gridDim.y, h = blockIdx.z;
    const int64_t th = (int64_t)h * nt + t;
    const int64_t tw = (int64_t)h * ntw + blockIdx.x;     // partial row of the tile
    const int64_t gs = (int64_t)h * ng + (t / group - g0);   // state / routing row: the tile's group
    const int r = w * 16 + col;                           // blockDim = 4 * tile: one wave per 16 rows
    const int64_t p = th * tile + r;
    i32x4 q8r[2], dq8r[2];
    load_row_ops(q8, dq8, p, grp, q8r, dq8r);
    const float sqr = sq[p], sdqr = sdq[p];
    RowState st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lo = sp * lps, hi = min(nb, lo + lps);
    const int e_n = kx * LEAF;
    const int e_lo = sp * eps, e_hi = min(e_n, e_lo + eps);
    tile_far_near<LEAF>(st, gs, nb, nb_pad, lo, hi, e_lo, e_hi, kx, q8r, sqr, dq8r, sdqr, g8, sg, lz,
                        vb, excl + gs * nb_pad, idx + gs * (kx > 0 ? kx : 1), k8, ks, v, (int64_t)h * nk, scale);
    const float ltot = grp_sum(st.l);
    if (pacc == nullptr) {   // single split: normalise in place
        const int64_t qi = (int64_t)t * tile + r;
        const int64_t oq = qi < nq ? perm_row(perm, h, nq, qi) : qi;
        write_final(st, ltot, (int64_t)h * nq + oq, qi < nq, out, logz);
        return;
    }
    const int64_t base = (tw * ns + sp) * tile + r;
    if (grp == 0) {
        pm[base] = st.m;
        pl[base] = ltot;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) *(f32x4*)(pacc + base * D + 16 * db + 4 * grp) = st.o[db];
}

// ---------------------------------------------------------------------------------------------
// 16-bit state stores, in the reference's stage structure:
//   fp8 (store="fp8", h3/htrc_flat_triton.py:65-72, 132-153, 214-254 with FP8 = 1):
//     select: SEL[g, l] = max_r (dq_r(fp16) . g_l(e4m3 -> fp16)) * sg_l + lz_l;
//     tile, far: score = (dq(fp16) . g) * sg + lz, O += (p * sv)(fp16) . vb(e4m3 -> fp16);
//   bf16 (store="bf16", DOT = 1 without FP8 / I8):
//     select: SEL = max_r dq_r(bf16) . g_l(bf16) + lz_l; far: score = dq . g + lz, O += p(bf16) . vb;
//   both, near: score = (q(bf16) . k(bf16)) * scale, O += p(bf16) . v(bf16).
// The e4m3 codes are widened to fp16 holding value * 2^-8 (e4m3x8_to_h8_cvt), exactly; sg and sv
// are taken times 256 (exact), so every product is the reference's.
// ---------------------------------------------------------------------------------------------
// QK A operand of state rows: 16 leaves x dims 32 ks + 8 grp .. + 7 of row `row`.
template <bool FP8>
__device__ __forceinline__ f32x4 state_qk(const void* g, int64_t row, int ks, int grp, const u32x4& b, f32x4 acc) {
    if constexpr (FP8)
        return mfma_f16(e4m3x8_to_h8_cvt(*(const u32x2*)((const uint8_t*)g + row * D + 32 * ks + 8 * grp)), b, acc);
    else
        return mfma_bf16(as_bf16x8(*(const u32x4*)((const uint16_t*)g + row * D + 32 * ks + 8 * grp)), as_bf16x8(b), acc);
}

template <bool FP8, int NRB>
__global__ __launch_bounds__(256) void select16_kernel(const uint16_t* __restrict__ dq16, int stride,
                                                       const void* __restrict__ g, const float* __restrict__ sg,
                                                       const float* __restrict__ lz, int nt, int group, int g0,
                                                       int ng, int nb, int nb_pad, float* __restrict__ sel) {
    constexpr int TR = 16 * NRB;                      // rows per tile
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int gi = blockIdx.x, h = blockIdx.z;
    const int64_t gs = (int64_t)h * ng + gi;          // state / SEL row of the group (the launch's window)
    const int ts = TR / stride;
    const int c0 = blockIdx.y * 256 + w * 64;
    float bsel[4][4];
#pragma unroll
    for (int lb = 0; lb < 4; ++lb)
#pragma unroll
        for (int i = 0; i < 4; ++i) bsel[lb][i] = -INFINITY;
    for (int j = 0; j < group; ++j) {
        const int t = (g0 + gi) * group + j;
        if (t >= nt) break;                           // padded tiles repeat the last one
        const int64_t th = (int64_t)h * nt + t;
        u32x4 b[NRB][4];
        bool val[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const int r = 16 * rb + col;
            val[rb] = r < ts;
            const int64_t p = th * TR + (int64_t)(val[rb] ? r : 0) * stride;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) b[rb][ks] = *(const u32x4*)(dq16 + p * D + 32 * ks + 8 * grp);
        }
#pragma unroll
        for (int lb = 0; lb < 4; ++lb) {
            const int c = c0 + 16 * lb;
            if (c < nb) {
                const int64_t s0 = gs * nb_pad + c;
                f32x4 acc[NRB];
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb) acc[rb] = state_qk<FP8>(g, s0 + col, ks, grp, b[rb][ks], acc[rb]);
                const f32x4 sgv = FP8 ? *(const f32x4*)(sg + s0 + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float best = -INFINITY;
                    const float sc = __fmul_rn(sgv[i], 256.0f);
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
                        best = fmaxf(best, FP8 ? __fmul_rn(acc[rb][i], sc) : acc[rb][i]);   // rows past ts repeat row 0
                    bsel[lb][i] = fmaxf(bsel[lb][i], col_max(best));
                }
            }
        }
    }
    if (col == 0) {
#pragma unroll
        for (int lb = 0; lb < 4; ++lb) {
            const int c = c0 + 16 * lb;
            if (c >= nb) break;
            const f32x4 lzv = *(const f32x4*)(lz + gs * nb_pad + c + 4 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int l = c + 4 * grp + i;
                if (l < nb) sel[gs * nb_pad + l] = __fadd_rn(bsel[lb][i], lzv[i]);
            }
        }
    }
}

// Online update (as online_block) whose PV operand is fp16: P = fp16(p * pscale) per key.
template <typename VFetch>
__device__ __forceinline__ void online_block_f16(RowState& st, float (&sc)[8], const float (&pscale)[8],
                                                 VFetch&& vfetch) {
    float bm = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) bm = fmaxf(bm, sc[e]);
    bm = grp_max(bm);
    const float m_new = fmaxf(st.m, bm);
    const float m_s = m_new == -INFINITY ? 0.0f : m_new;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = __expf(__fsub_rn(sc[e], m_s));
        ps = __fadd_rn(ps, p[e]);
    }
    const float alpha = __expf(__fsub_rn(st.m, m_s));
    st.l = __fadd_rn(__fmul_rn(st.l, alpha), ps);
    uint32_t ph[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        ph[j] = pack2h(__fmul_rn(p[2 * j], pscale[2 * j]), __fmul_rn(p[2 * j + 1], pscale[2 * j + 1]));
    const u32x4 P = u32x4{ph[0], ph[1], ph[2], ph[3]};
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        f32x4 o = st.o[db];
        o[0] = __fmul_rn(o[0], alpha);
        o[1] = __fmul_rn(o[1], alpha);
        o[2] = __fmul_rn(o[2], alpha);
        o[3] = __fmul_rn(o[3], alpha);
        st.o[db] = mfma_f16(vfetch(db), P, o);
    }
    st.m = m_new;
}

template <int LEAF, bool FP8>
__global__ __launch_bounds__(256) void tile16_kernel(
    const uint16_t* __restrict__ q16, const uint16_t* __restrict__ dq16, const void* __restrict__ g,
    const float* __restrict__ sg, const float* __restrict__ lz, const void* __restrict__ vb,
    const float* __restrict__ sv, const int8_t* __restrict__ excl, const int32_t* __restrict__ idx,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t nq, int nt, int tile, int group,
    int g0, int ng, const int32_t* __restrict__ perm, int64_t nk, int nb, int nb_pad, int kx, int lps, int eps,
    float scale, float* __restrict__ pm, float* __restrict__ pl, float* __restrict__ pacc, float* __restrict__ out,
    float* __restrict__ logz) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // tiles of groups [g0, g0 + ng): state, routing and partial rows are the launch's own
    const int tb = g0 * group, ntw = gridDim.x;
    const int t = tb + blockIdx.x, sp = blockIdx.y, ns = gridDim.y, h = blockIdx.z;
    const int64_t th = (int64_t)h * nt + t;
    const int64_t tw = (int64_t)h * ntw + blockIdx.x;     // partial row of the tile
    const int64_t gs = (int64_t)h * ng + (t / group - g0);   // state / routing row: the tile's group
    const int r = w * 16 + col;                           // blockDim = 4 * tile: one wave per 16 rows
    const int64_t p = th * tile + r;
    u32x4 qb[4], dqh[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        qb[ks] = *(const u32x4*)(q16 + p * D + 32 * ks + 8 * grp);
        dqh[ks] = *(const u32x4*)(dq16 + p * D + 32 * ks + 8 * grp);
    }
    RowState st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int lo = sp * lps, hi = min(nb, lo + lps);
    const int e_n = kx * LEAF;
    const int e_lo = sp * eps, e_hi = min(e_n, e_lo + eps);
    const int8_t* excl_row = excl + gs * nb_pad;
    // ---- far field
    for (int c0 = lo; c0 < hi; c0 += 32) {
        float sc[8], pscale[8];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int cb = c0 + 16 * h2;
            const int64_t s0 = gs * nb_pad + cb;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) acc = state_qk<FP8>(g, s0 + col, ks, grp, dqh[ks], acc);
            const f32x4 sgv = FP8 ? *(const f32x4*)(sg + s0 + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
            const f32x4 svv = FP8 ? *(const f32x4*)(sv + s0 + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
            const f32x4 lzv = *(const f32x4*)(lz + s0 + 4 * grp);
            const uint32_t exv = *(const uint32_t*)(excl_row + cb + 4 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = cb + 4 * grp + i;
                const bool ok = c < hi && ((exv >> (8 * i)) & 0xffu) == 0u;
                const float dot = FP8 ? __fmul_rn(acc[i], __fmul_rn(sgv[i], 256.0f)) : acc[i];
                sc[4 * h2 + i] = ok ? __fadd_rn(dot, lzv[i]) : -INFINITY;
                pscale[4 * h2 + i] = __fmul_rn(svv[i], 256.0f);
            }
        }
        if constexpr (FP8) {
            const uint8_t* vb0 = (const uint8_t*)vb + (gs * nb_pad + c0) * D;
            online_block_f16(st, sc, pscale, [&](int db) {   // vb^T: keys 4grp + j and 16 + 4grp + j at one dim
                const int dim = 16 * db + col;
                uint32_t u[2];
#pragma unroll
                for (int jh = 0; jh < 2; ++jh) {
                    const uint8_t* b = vb0 + (16 * jh + 4 * grp) * D + dim;
                    u[jh] = (uint32_t)b[0] | ((uint32_t)b[D] << 8) | ((uint32_t)b[2 * D] << 16) |
                            ((uint32_t)b[3 * D] << 24);
                }
                return e4m3x8_to_h8_cvt(u32x2{u[0], u[1]});
            });
        } else {
            const uint16_t* vb0 = (const uint16_t*)vb + (gs * nb_pad + c0) * D;
            online_block(st, sc, [&](int db) { return gather_pv(vb0, 0, 16, 16 * db + col, grp); });
        }
    }
    // ---- near field: token j of the tile's selected list -> idx[j / LEAF] * LEAF + j % LEAF
    const int32_t* idx_row = idx + gs * (kx > 0 ? kx : 1);
    const int64_t kh = (int64_t)h * nk;
    for (int e0 = e_lo; e0 < e_hi; e0 += 32) {
        float sc[8];
        int64_t tok0[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int j0 = e0 + 16 * h2;
            const bool ok = j0 < e_hi;
            const int jj = ok ? j0 : e_lo;
            tok0[h2] = kh + (int64_t)idx_row[jj / LEAF] * LEAF + (jj % LEAF);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                acc = mfma_bf16(as_bf16x8(*(const u32x4*)(k + (tok0[h2] + col) * D + 32 * ks + 8 * grp)),
                                as_bf16x8(qb[ks]), acc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool oki = ok && (j0 + 4 * grp + i) < e_hi;
                sc[4 * h2 + i] = oki ? __fmul_rn(acc[i], scale) : -INFINITY;
            }
        }
        online_block(st, sc, [&](int db) { return gather_pv(v, tok0[0], tok0[1], 16 * db + col, grp); });
    }
    const float ltot = grp_sum(st.l);
    if (pacc == nullptr) {   // single split: normalise in place
        const int64_t qi = (int64_t)t * tile + r;
        const int64_t oq = qi < nq ? perm_row(perm, h, nq, qi) : qi;
        write_final(st, ltot, (int64_t)h * nq + oq, qi < nq, out, logz);
        return;
    }
    const int64_t base = (tw * ns + sp) * tile + r;
    if (grp == 0) {
        pm[base] = st.m;
        pl[base] = ltot;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) *(f32x4*)(pacc + base * D + 16 * db + 4 * grp) = st.o[db];
}

// ---------------------------------------------------------------------------------------------
// fp32 dots (dot other than "bf16": h3/htrc_flat_triton.py:138-141, 159-161, 171-174, 184-185,
// 245-247 with DOT = 0): the state g, vb in fp32 (store="fp32") or bf16 (store="bf16", widened
// exactly), q and q - mu in fp32, k and v the bf16 keys / values widened exactly; every product
// by the fp32 MFMA (v_mfma_f32_16x16x4_f32) with fp32 sums.  TF32 (precision="tf32", the
// reference's PREC "tf32"): every operand is first rounded to TF32 (tf32_rna), whose products
// fp32 holds exactly.
// 16x16x4 operands: lane l supplies A[m = l%16][k = l/16] and B[k = l/16][n = l%16].  In a QK
// product, step s (0..31) lets k-index l/16 stand for dim 32 (l/16) + s, so each lane holds 32
// consecutive dims of its key row (A) and of its query row (B).  In a PV product over 16 keys,
// step s lets it stand for key 4 (l/16) + s, which is item s of the lane's score tile C[4 (l/16)
// + i][l%16] (no shuffle), and row m of the O^T block db stands for dim 8 m + db, so the A
// operand is 8 consecutive dims of a value row and the lane's O^T items are dims 32 (l/16) ..
// + 31 of its query row.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// N consecutive values (bf16 when BF, else fp32) from p, as fp32; TF32-rounded when TF32 (a
// no-op on bf16 values, which TF32 holds).
template <int N, bool BF, bool TF32>
__device__ __forceinline__ void load_f32(const void* p, float (&x)[N]) {
    static_assert(N % 8 == 0, "load_f32: whole 16-byte pieces");
    if constexpr (BF) {
#pragma unroll
        for (int q = 0; q < N / 8; ++q) {
            const u32x4 u = ((const u32x4*)p)[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[8 * q + 2 * e] = bf2f(u[e] & 0xffffu);
                x[8 * q + 2 * e + 1] = bf2f(u[e] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
            const f32x4 f = ((const f32x4*)p)[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * q + e] = TF32 ? tf32_rna(f[e]) : f[e];
        }
    }
}

// x (8 floats) as n bf16 terms whose sum is x exactly: each term the bf16 rounding of what the
// terms before it leave (that residual is exact in fp32); n = 3 holds any fp32 value, n = 2 a
// TF32 one, n = 1 a bf16 one.  x is consumed.
__device__ __forceinline__ void split_terms(float (&x)[8], bf16x8 (&t)[3], int n) {
#pragma unroll
    for (int tt = 0; tt < 3; ++tt) {
        if (tt >= n) break;
        const u32x4 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3]), pack2bf(x[4], x[5]), pack2bf(x[6], x[7])};
        t[tt] = as_bf16x8(u);
        if (tt + 1 < n) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = __fsub_rn(x[2 * e], __uint_as_float(u[e] << 16));
                x[2 * e + 1] = __fsub_rn(x[2 * e + 1], __uint_as_float(u[e] & 0xffff0000u));
            }
        }
    }
}
// 16x16x16 bf16 MFMA: a and b hold 4 bf16 each (A[l % 16][4 (l / 16) + j], B[4 (l / 16) + j][l % 16])
__device__ __forceinline__ f32x4 mfma_bf16_k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0,
                                                      0, 0);
}

struct RowF32 {        // running softmax state of one row (h3/htrc_flat_triton.py:142-157)
    float m;           // running max (natural log units; the same in the four lanes of a row)
    float l;           // this lane's share of the running sum
    f32x4 o[8];        // O^T: item i of block db is dim 16 db + 4 grp + i (the fp32-MFMA far
                       // field keeps dim 8 (4 grp + i) + db and reorders once, before the near field)
};

// One block of 16 keys: scores sc[i] of keys 4 grp + i (masked: -inf), value rows va[s] = dims
// 8 col .. + 7 of key 4 grp + s.  The reference's update: m_new = max(m, rowmax), m_s = m_new, or
// 0 when -inf, p = exp(sc - m_s), alpha = exp(m - m_s), l = l alpha + sum p, O = O alpha + P V.
template <bool TF32>
__device__ __forceinline__ void f32_update(RowF32& st, const float (&sc)[4], const float (&va)[4][8]) {
    const float bm = grp_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float mn = fmaxf(st.m, bm);
    const float ms = mn == -INFINITY ? 0.0f : mn;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __expf(__fsub_rn(sc[i], ms));
    const float alpha = __expf(__fsub_rn(st.m, ms));
    st.l = __fadd_rn(__fmul_rn(st.l, alpha), __fadd_rn(__fadd_rn(p[0], p[1]), __fadd_rn(p[2], p[3])));
    // O alpha: skipped when every row's alpha is 1 (no running maximum moved: the same bits)
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) st.o[db][i] = __fmul_rn(st.o[db][i], alpha);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float ps = TF32 ? tf32_rna(p[s]) : p[s];
#pragma unroll
        for (int db = 0; db < 8; ++db) st.o[db] = mfma_f32(va[s][db], ps, st.o[db]);
    }
    st.m = mn;
}


// Far + near field of one (tile, split) with fp32 dots (h3/htrc_flat_triton.py:88-211, DOT = 0):
// far leaves [sp lps, + lps) not excluded, score = (q - mu) . g + lz; near tokens [sp eps, + eps)
// of the tile group's idx leaves, score = (q . k) scale.  One wave per 16 rows; the workgroup
// stages each block's state rows, and the near field's key and value rows, in LDS once for all
// its waves.  ns == 1 (pacc null): normalised rows and logz = m + log l; else the partial
// (m, l, O) for merge_kernel.
template <bool QBF, bool SB, bool TF32>
__global__ __launch_bounds__(256, 3) void tile_f32_kernel(
    const void* __restrict__ q, const float* __restrict__ mu, int mu_stride, const void* __restrict__ g,
    const float* __restrict__ lz, const void* __restrict__ vb, const int8_t* __restrict__ excl,
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t nq,
    int nt, int tile, int group, int g0, int ng, const int32_t* __restrict__ perm, int64_t nk, int leaf, int nb,
    int nb_pad, int kx, int lps, int eps, float scale, float* __restrict__ pm, float* __restrict__ pl,
    float* __restrict__ pacc, float* __restrict__ out, float* __restrict__ logz) {
    constexpr int QB = QBF ? 2 : 4, SBB = SB ? 2 : 4;          // bytes per value
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, col = lane & 15,
              grp = lane >> 4;
    const int tb = g0 * group, ntw = gridDim.x;
    const int t = tb + blockIdx.x, sp = blockIdx.y, ns = gridDim.y, h = blockIdx.z;
    const int64_t tw = (int64_t)h * ntw + blockIdx.x;         // partial row of the tile
    const int64_t gs = (int64_t)h * ng + (t / group - g0);    // state / routing row: the tile's group
    const int r = 16 * w + col;                                // blockDim = 4 * tile: one wave per 16 rows
    const int64_t qi = (int64_t)t * tile + r;                  // pad rows repeat the last query
    const int64_t src = perm_row(perm, h, nq, qi < nq ? qi : nq - 1);
    // Products on the bf16 MFMA over exact bf16 terms (split_terms): a state value (g, vb) in NGT
    // terms, q - mu in ND, a far weight in NPF, so every product is the exact product the fp32
    // MFMA forms and only the grouping of the fp32 sums differs.
    constexpr int NGT = SB ? 1 : (TF32 ? 2 : 3), ND = TF32 ? 2 : 3, NPF = TF32 ? 2 : 3;
    // The far field takes these products for TF32 operands and bf16 rows; for IEEE operands on
    // fp32 rows only its scores do (g in three terms), and its PV products run on the fp32 MFMA
    // (v_mfma_f32_16x16x4_f32), which measured faster there: three terms of every vb value cost
    // more splitting than their products save.
    constexpr bool FTERMS = TF32 || SB;
    // q - mu of row r in ND terms: k-step ks holds lane group grp's dims 32 ks + 8 grp .. + 7
    bf16x8 dqt[4][3];
    {
        const char* qrow = (const char*)q + ((int64_t)h * nq + src) * D * QB;
        const float* murow = mu + ((int64_t)h * mu_stride + t / group) * D + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float x[8], mx[8];
            load_f32<8, QBF, false>(qrow + (32 * ks + 8 * grp) * QB, x);
            load_f32<8, false, false>(murow + 32 * ks, mx);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x[e] = __fsub_rn(x[e], mx[e]);
                if constexpr (TF32) x[e] = tf32_rna(x[e]);
            }
            split_terms(x, dqt[ks], ND);
        }
    }
    RowF32 st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    // ---- far field: 16 leaves per block.  The block's state rows reach a raw slot in LDS by
    // direct loads (g rows, vb rows, lz, the exclusion bytes; row r keeps its 16-byte chunk c at
    // c ^ r); the workgroup then splits them once into bf16 terms (g term rows with chunk c at
    // c ^ leaf, for the score operands; vb term rows with chunk c at c ^ swz(leaf), for the
    // transposing PV reads) and loads the next block into the raw slot while its waves take
    // their products from the terms.  The near field reuses the buffer as two key + value slots.
    constexpr int RBY = D * SBB;                   // state row bytes: 512 (fp32) or 256 (bf16)
    constexpr int CR = RBY / 16;                   // chunks per row: 32 or 16
    constexpr int GV = 16 * RBY;                   // g rows of a block; the vb rows follow
    constexpr int RAW = 2 * GV + 128;              // raw slot: g, vb rows, lz (64 B), exclusion bytes
    constexpr int TB = 16 * 256;                   // one term of 16 leaf rows (bf16)
    constexpr int NSLOT = 16384;                   // near field slot: 32 key rows, 32 value rows
    constexpr int FSLOT = RAW;                     // fp32-MFMA far field: two raw slots, no terms
    constexpr int LDSZ_T = RAW + 2 * NGT * TB + 128 > 2 * NSLOT ? RAW + 2 * NGT * TB + 128 : 2 * NSLOT;
    constexpr int LDSZ = FTERMS ? LDSZ_T : 2 * FSLOT + NGT * TB;   // (2 FSLOT > 2 NSLOT)
    __shared__ __align__(16) char lbuf[LDSZ];
    char* const tgs = lbuf + RAW;                  // g terms
    char* const tvs = tgs + NGT * TB;              // vb terms
    char* const taux = tvs + NGT * TB;             // the block's lz (16 floats) and exclusion bytes
    const int lo = sp * lps, hi = min(nb, lo + lps);
    const int64_t srow = gs * nb_pad;
    const int nblk = hi > lo ? (hi - lo + 15) / 16 : 0;
    const int nw = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);   // waves: 4 (64-row tiles) or 2
    const int tid = threadIdx.x, nth = blockDim.x;
    const uint32_t lbuf_lds = lds_addr(lbuf);
    // block bi into the raw slot: instruction i (NI per matrix: g rows, then vb rows) loads chunks
    // p = 64 i' + lane of its matrix (i' = i mod NI): row p / CR, chunk (p % CR) ^ row, from the
    // block's first row (wave-uniform, in SGPRs) plus a 32-bit lane offset.  Wave w issues
    // instructions w, w + nw, ..; rows up to c0 + 15 < nb_pad exist in the state (nb_pad is a
    // multiple of 32, c0 of 16; rows past nb hold the zero state of padded leaves), those past
    // hi are masked.
    constexpr int NI = GV / 1024;
    const int lr = lane / CR, lc = lane % CR;
    auto far_issue = [&](int bi, uint32_t dst) {
        const int c0 = lo + 16 * bi;
        const char* gb = (const char*)g + (srow + c0) * RBY;
        const char* vbb = (const char*)vb + (srow + c0) * RBY;
        int lrx = lr;
        asm volatile("" : "+v"(lrx));          // the lane offsets computed here, not held across the loop
#pragma unroll
        for (int j = 0; j < NI; ++j) {         // nw >= 2: at most NI instructions per wave
            const int i = w + nw * j;
            if (i >= 2 * NI) break;
            const int r = (64 / CR) * (i >= NI ? i - NI : i) + lrx;
            dma16s(i >= NI ? vbb : gb, (uint32_t)(r * RBY + ((lc ^ r) << 4)), dst + 1024 * i);
        }
        if (w == 0 && lane < 5)        // lz of the 16 leaves (lanes 0..3), their exclusion bytes (4)
            dma16(lane < 4 ? (const void*)(lz + srow + c0 + 4 * lane) : (const void*)(excl + srow + c0),
                  dst + 2 * GV);
    };
    // raw slot -> terms: unit u = leaf u / 16, dims 8 (u % 16) .. + 7 of g and of vb (TF32: each
    // value rounded first); the lz and exclusion bytes copied beside the terms
    auto far_split = [&]() {
        for (int u = tid; u < 256; u += nth) {
            const int lf = u >> 4, c = u & 15;
#pragma unroll
            for (int mtx = 0; mtx < 2; ++mtx) {
                const char* row = lbuf + mtx * GV + lf * RBY;
                float x[8];
                if constexpr (SB) {
                    const u32x4 raw = *(const u32x4*)(row + ((c ^ lf) << 4));
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        x[2 * e] = bf2f(raw[e] & 0xffffu);
                        x[2 * e + 1] = bf2f(raw[e] >> 16);
                    }
                } else {
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const f32x4 f = *(const f32x4*)(row + (((2 * c + hf) ^ lf) << 4));
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[4 * hf + e] = TF32 ? tf32_rna(f[e]) : f[e];
                    }
                }
                bf16x8 tt[3];
                split_terms(x, tt, NGT);
                char* dst = mtx == 0 ? tgs + lf * 256 + ((c ^ lf) << 4) : tvs + lf * 256 + ((c ^ swz(lf)) << 4);
#pragma unroll
                for (int a = 0; a < NGT; ++a) *(bf16x8*)(dst + a * TB) = tt[a];
            }
        }
        if (tid < 5) *(u32x4*)(taux + 16 * tid) = *(const u32x4*)(lbuf + 2 * GV + 16 * tid);
    };
    // the reference's update over the block (h3/htrc_flat_triton.py:142-157): m_new = max(m,
    // rowmax), m_s = m_new or 0 when -inf, p = exp(sc - m_s), alpha = exp(m - m_s), l = l alpha +
    // sum p, O = O alpha + P V
    auto far_block = [&](int bi) {
        const int c0 = lo + 16 * bi;
        // S^T: leaf 4 grp + i, row col (g terms as A, q - mu terms as B), smaller products first
        f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sum = NGT + ND - 2; sum >= 0; --sum)
#pragma unroll
            for (int a = 0; a < NGT; ++a) {
                const int b = sum - a;
                if (b < 0 || b >= ND) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const bf16x8 ga = *(const bf16x8*)(tgs + a * TB + col * 256 + (((4 * ks + grp) ^ col) << 4));
                    s4 = mfma_bf16(ga, dqt[ks][b], s4);
                }
            }
        const f32x4 lz4 = *(const f32x4*)(taux + 16 * grp);
        const uint32_t ex4 = *(const uint32_t*)(taux + 64 + 4 * grp);
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + 4 * grp + i;
            sc[i] = (c < hi && ((ex4 >> (8 * i)) & 0xffu) == 0) ? __fadd_rn(s4[i], lz4[i]) : -INFINITY;
        }
        const float bm = grp_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        const float mn = fmaxf(st.m, bm);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = __expf(__fsub_rn(sc[i], ms));
        const float alpha = __expf(__fsub_rn(st.m, ms));
        st.l = __fadd_rn(__fmul_rn(st.l, alpha), __fadd_rn(__fadd_rn(pr[0], pr[1]), __fadd_rn(pr[2], pr[3])));
        // O alpha: skipped when every row's alpha is 1 (no running maximum moved: the same bits)
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) st.o[db][i] = __fmul_rn(st.o[db][i], alpha);
        }
        st.m = mn;
        // the weights (TF32-rounded for TF32 operands) as NPF bf16 terms: B of the 16x16x16
        // products, k = leaf 4 grp + j
        u32x2 pt[3];
        {
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = TF32 ? tf32_rna(pr[i]) : pr[i];
#pragma unroll
            for (int tt = 0; tt < NPF; ++tt) {
                const u32x2 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3])};
                pt[tt] = u;
                if (tt + 1 < NPF) {
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        x[2 * e] = __fsub_rn(x[2 * e], __uint_as_float(u[e] << 16));
                        x[2 * e + 1] = __fsub_rn(x[2 * e + 1], __uint_as_float(u[e] & 0xffff0000u));
                    }
                }
            }
        }
        // O^T += vb^T P^T: A = vb terms by transposing reads (leaves 4 grp + j, dim 16 db + col)
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int sum = NGT + NPF - 2; sum >= 0; --sum)
#pragma unroll
                for (int a = 0; a < NGT; ++a) {
                    const int b = sum - a;
                    if (b < 0 || b >= NPF) continue;
                    st.o[db] = mfma_bf16_k16(tr_operand(tvs + a * TB, 0, db, lane), pt[b], st.o[db]);
                }
    };
    // IEEE operands on fp32 rows: two raw slots, the next block's loads issued before this
    // block's work; the workgroup splits the block's g rows once into three bf16 terms (after
    // the raw slots) for the score products, and the PV products run on the fp32 MFMA with each
    // wave reading its vb operands from the raw rows (dims 8 col .. of rows 4 grp + s)
    char* const tg3 = lbuf + 2 * FSLOT;
    auto far_split_g = [&](int slot) {
        for (int u = tid; u < 256; u += nth) {
            const int lf = u >> 4, c = u & 15;
            const char* row = lbuf + slot * FSLOT + lf * RBY;
            float x[8];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const f32x4 f = *(const f32x4*)(row + (((2 * c + hf) ^ lf) << 4));
#pragma unroll
                for (int e = 0; e < 4; ++e) x[4 * hf + e] = f[e];
            }
            bf16x8 tt[3];
            split_terms(x, tt, NGT);
#pragma unroll
            for (int a = 0; a < NGT; ++a) *(bf16x8*)(tg3 + a * TB + lf * 256 + ((c ^ lf) << 4)) = tt[a];
        }
    };
    auto far_block_f32 = [&](int bi, int slot) {
        const int c0 = lo + 16 * bi;
        const char* sl = lbuf + slot * FSLOT;
        float va[4][8];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int rr = 4 * grp + s2;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const f32x4 f = *(const f32x4*)(sl + GV + rr * RBY + (((2 * col + hf) ^ rr) << 4));
#pragma unroll
                for (int e = 0; e < 4; ++e) va[s2][4 * hf + e] = f[e];
            }
        }
        const f32x4 lz4 = *(const f32x4*)(sl + 2 * GV + 16 * grp);
        const uint32_t ex4 = *(const uint32_t*)(sl + 2 * GV + 64 + 4 * grp);
        // (k-step by k-step: the step's three g terms held, its nine products smallest first)
        f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 ga[3];
#pragma unroll
            for (int a = 0; a < NGT; ++a)
                ga[a] = *(const bf16x8*)(tg3 + a * TB + col * 256 + (((4 * ks + grp) ^ col) << 4));
#pragma unroll
            for (int sum = NGT + ND - 2; sum >= 0; --sum)
#pragma unroll
                for (int a = 0; a < NGT; ++a) {
                    const int b = sum - a;
                    if (b >= 0 && b < ND) s4 = mfma_bf16(ga[a], dqt[ks][b], s4);
                }
        }
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + 4 * grp + i;
            sc[i] = (c < hi && ((ex4 >> (8 * i)) & 0xffu) == 0) ? __fadd_rn(s4[i], lz4[i]) : -INFINITY;
        }
        f32_update<false>(st, sc, va);
    };
    if constexpr (FTERMS) {
        if (nblk > 0) far_issue(0, lbuf_lds);
        for (int bi = 0; bi < nblk; ++bi) {
            wait_vmcnt<0>();                       // this wave's loads of block bi have landed
            __syncthreads();                       // every wave's; every wave done with the terms
            far_split();
            __syncthreads();                       // the terms complete; the raw slot is free
            if (bi + 1 < nblk) far_issue(bi + 1, lbuf_lds);
            far_block(bi);
        }
    } else {
        if (nblk > 0) far_issue(0, lbuf_lds);
        for (int bi = 0; bi < nblk; ++bi) {
            wait_vmcnt<0>();                       // this wave's loads of block bi have landed
            __syncthreads();                       // every wave's; slot (bi + 1) & 1 and the terms free
            if (bi + 1 < nblk) far_issue(bi + 1, lbuf_lds + (uint32_t)(((bi + 1) & 1) * FSLOT));
            far_split_g(bi & 1);
            __syncthreads();                       // the g terms complete
            far_block_f32(bi, bi & 1);
        }
    }
    // Near-field score operands on the bf16 MFMA (16x16x32): k-step s takes lane group grp's dims
    // 32 s + 8 grp .. + 7 of the row as NQT bf16 terms whose sum is the row exactly (a bf16 row:
    // itself; TF32: 11 bits in two; fp32: 24 bits in three, each residual exact), so every product
    // with a bf16 key is the exact product the fp32 MFMA forms and only the grouping of the fp32
    // sums differs, at a quarter (fp32 rows) to an eighth (bf16 rows) of its matrix cycles.
    constexpr int NQT = QBF ? 1 : (TF32 ? 2 : 3);
    bf16x8 qt[NQT][4];
    {
        const char* qrow = (const char*)q + ((int64_t)h * nq + src) * D * QB;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float x[8];
            load_f32<8, QBF, false>(qrow + (32 * ks + 8 * grp) * QB, x);
#pragma unroll
            for (int tt = 0; tt < NQT; ++tt) {
                if constexpr (TF32) {
                    if (tt == 0) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = tf32_rna(x[e]);
                    }
                }
                const u32x4 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3]), pack2bf(x[4], x[5]), pack2bf(x[6], x[7])};
                qt[tt][ks] = as_bf16x8(u);
                if (tt + 1 < NQT) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {       // the residual, exact
                        x[2 * e] = __fsub_rn(x[2 * e], __uint_as_float(u[e] << 16));
                        x[2 * e + 1] = __fsub_rn(x[2 * e + 1], __uint_as_float(u[e] & 0xffff0000u));
                    }
                }
            }
        }
    }
    // ---- near field: 32 tokens per block, on the bf16 MFMA.  Scores in two 16-key halves (the
    // lane's keys 4 grp + i and 16 + 4 grp + i of the block); the PV products take the block's
    // values from LDS by transposing reads (O^T item i of block db: dim 16 db + 4 grp + i) and
    // the weights as NPT bf16 terms that sum to them exactly (each product with a bf16 value
    // exact, as in the fp32 MFMA).  The block's running maximum is taken over its 32 keys (the
    // reference's block size is a launch parameter).
    constexpr int NPT = TF32 ? 2 : 3;
    const int e_n = kx * leaf;
    const int e_lo = sp * eps, e_hi = min(e_n, e_lo + eps);
    const int64_t kh = (int64_t)h * nk;
    const int32_t* ix = idx + gs * (int64_t)(kx > 0 ? kx : 1);
    // a block's two 16-token runs (each in one leaf: leaf, e_lo and the split length are
    // multiples of 16): wave-uniform bases, and the last valid position of each (a run past e_hi
    // repeats the first run, masked)
    struct Runs {
        int64_t b[2];
        int last[2];
    };
    const int lsh = __builtin_ctz(leaf);        // leaf is a power of two
    auto runs = [&](int e0) {
        Runs r;
        r.b[0] = kh + (int64_t)ix[e0 >> lsh] * leaf + (e0 & (leaf - 1));
        r.last[0] = min(15, e_hi - 1 - e0);
        if (e0 + 16 < e_hi) {
            r.b[1] = kh + (int64_t)ix[(e0 + 16) >> lsh] * leaf + ((e0 + 16) & (leaf - 1));
            r.last[1] = min(15, e_hi - 17 - e0);
        } else {
            r.b[1] = r.b[0];
            r.last[1] = -1;
        }
        return r;
    };
    __syncthreads();                            // every wave done with the far field's buffer
    if constexpr (!FTERMS) {
        // the fp32-MFMA far field's accumulators to the near field's order, through this wave's
        // 8 KB of the buffer (row col, 16-byte chunk c at c ^ col): far order dims 32 grp + 8 i +
        // 4 hf .. + 3 (chunk 8 grp + 2 i + hf) = st.o[4 hf .. 4 hf + 3][i]; near order dims 16 db +
        // 4 grp .. + 3 (chunk 4 db + grp) = st.o[db]
        char* tw_ = lbuf + w * 8192;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                *(f32x4*)(tw_ + col * 512 + (((8 * grp + 2 * i + hf) ^ col) << 4)) =
                    f32x4{st.o[4 * hf][i], st.o[4 * hf + 1][i], st.o[4 * hf + 2][i], st.o[4 * hf + 3][i]};
        __syncthreads();
#pragma unroll
        for (int db = 0; db < 8; ++db) st.o[db] = *(const f32x4*)(tw_ + col * 512 + (((4 * db + grp) ^ col) << 4));
        __syncthreads();                        // every wave's accumulators read: the buffer is free
    }
    // a block's 32 key rows (bytes 0.., chunk c of row r at c ^ (r % 16), so the 16 lanes that
    // read one chunk of 16 rows address 16 positions) and its 32 value rows (bytes 8192.., chunk
    // c of row r at c ^ swz(r), the transposing reads' layout) into a slot of the shared buffer
    // by direct loads; a row past its run's last valid position repeats that position's token
    // (instruction i: keys for i < 8, values after; its rows 4 (i % 8) + lane / 16, in run
    // hh = (i % 8) / 4, wave-uniform; the run's first token in SGPRs, a 32-bit lane offset)
    auto kvload = [&](const Runs& rr, int slot) {
        const uint32_t sl = lbuf_lds + (uint32_t)(slot * NSLOT);
#pragma unroll
        for (int j = 0; j < 8; ++j) {           // nw >= 2: at most 8 instructions per wave
            const int i = w + nw * j;
            if (i >= 16) break;
            const int isv = i >> 3, ii = i & 7, hh = ii >> 2;
            const int rw = 4 * (ii & 3) + (lane >> 4);       // row % 16
            const int lst = hh ? (rr.last[1] >= 0 ? rr.last[1] : rr.last[0]) : rr.last[0];
            const int c = (lane & 15) ^ (isv ? swz(rw) : rw);
            dma16s((isv ? v : k) + (hh ? rr.b[1] : rr.b[0]) * D, (uint32_t)(min(rw, lst) * 256 + (c << 4)),
                   sl + 1024 * i);
        }
    };
    // run bases one block ahead of the loads that use them (their index reads then land under
    // a block's products instead of delaying the next block's loads)
    Runs rn{}, rn1{};
    if (e_lo < e_hi) {
        rn = runs(e_lo);
        kvload(rn, 0);
        if (e_lo + 32 < e_hi) rn1 = runs(e_lo + 32);
    }
    int kslot = 0;
    for (int e0 = e_lo; e0 < e_hi; e0 += 32, kslot ^= 1) {
        const Runs cur = rn;
        wait_vmcnt<0>();                        // this wave's loads of the block have landed
        __syncthreads();                        // every wave's; the other slot is free
        if (e0 + 32 < e_hi) {                   // the next block loads under this one
            rn = rn1;
            kvload(rn, kslot ^ 1);
            if (e0 + 64 < e_hi) rn1 = runs(e0 + 64);
        }
        const char* ks_ = lbuf + kslot * NSLOT;
        const char* vs_ = ks_ + 8192;
        float sc[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            u32x4 kq[4];
            const int krw = 16 * hh + col;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kq[ks] = *(const u32x4*)(ks_ + krw * 256 + (((4 * ks + grp) ^ col) << 4));
            f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int tt = NQT - 1; tt >= 0; --tt)        // smaller terms first
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) s4 = mfma_bf16(as_bf16x8(kq[ks]), qt[tt][ks], s4);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                sc[4 * hh + i] = 4 * grp + i <= cur.last[hh] ? __fmul_rn(s4[i], scale) : -INFINITY;
        }
        // the reference's update over the block: m_new = max(m, rowmax), m_s = m_new or 0 when
        // -inf, p = exp(sc - m_s), alpha = exp(m - m_s), l = l alpha + sum p, O = O alpha + P V
        float bm = sc[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) bm = fmaxf(bm, sc[i]);
        bm = grp_max(bm);
        const float mn = fmaxf(st.m, bm);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pr[i] = __expf(__fsub_rn(sc[i], ms));
        const float alpha = __expf(__fsub_rn(st.m, ms));
        st.l = __fadd_rn(__fmul_rn(st.l, alpha),
                         __fadd_rn(__fadd_rn(__fadd_rn(pr[0], pr[1]), __fadd_rn(pr[2], pr[3])),
                                   __fadd_rn(__fadd_rn(pr[4], pr[5]), __fadd_rn(pr[6], pr[7]))));
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int db = 0; db < 8; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) st.o[db][i] = __fmul_rn(st.o[db][i], alpha);
        }
        st.m = mn;
        // the weights (TF32-rounded for TF32 operands) as NPT bf16 terms, k slot j of lane group
        // grp = key 4 grp + j (j < 4) or 16 + 4 grp + j - 4
        bf16x8 pt[NPT];
        {
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = TF32 ? tf32_rna(pr[i]) : pr[i];
#pragma unroll
            for (int tt = 0; tt < NPT; ++tt) {
                const u32x4 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3]), pack2bf(x[4], x[5]), pack2bf(x[6], x[7])};
                pt[tt] = as_bf16x8(u);
                if (tt + 1 < NPT) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        x[2 * e] = __fsub_rn(x[2 * e], __uint_as_float(u[e] << 16));
                        x[2 * e + 1] = __fsub_rn(x[2 * e + 1], __uint_as_float(u[e] & 0xffff0000u));
                    }
                }
            }
        }
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const u32x2 a0 = tr_operand(vs_, 0, db, lane), a1 = tr_operand(vs_, 16, db, lane);
            const bf16x8 A = as_bf16x8(a0, a1);
#pragma unroll
            for (int tt = NPT - 1; tt >= 0; --tt) st.o[db] = mfma_bf16(A, pt[tt], st.o[db]);
        }
    }
    const float ltot = grp_sum(st.l);
    // the lane's O^T items: dims 16 db + 4 grp .. + 3 are st.o[db]
    if (pacc == nullptr) {                                     // single split: normalise in place
        int rx = r;
        asm volatile("" : "+v"(rx));           // the row index recomputed here, not held across the loops
        const int64_t qo = (int64_t)t * tile + rx;
        if (qo >= nq) return;
        const int64_t orow = (int64_t)h * nq + perm_row(perm, h, nq, qo);
        const float ms = st.m == -INFINITY ? 0.0f : st.m;
        const float den = ltot < 1e-30f ? 1e-30f : ltot;
#pragma unroll
        for (int db = 0; db < 8; ++db)
            *(f32x4*)(out + orow * D + 16 * db + 4 * grp) =
                f32x4{__fdiv_rn(st.o[db][0], den), __fdiv_rn(st.o[db][1], den), __fdiv_rn(st.o[db][2], den),
                      __fdiv_rn(st.o[db][3], den)};
        if (grp == 0) logz[orow] = __fadd_rn(ms, __logf(ltot));
        return;
    }
    const int64_t base = (tw * ns + sp) * tile + r;
    if (grp == 0) {
        pm[base] = st.m;
        pl[base] = ltot;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) *(f32x4*)(pacc + base * D + 16 * db + 4 * grp) = st.o[db];
}

// SEL[g, l] = max over every stride-th row of the group's tiles of (q - mu_g) . g_l, + lz_l, with
// fp32 dots (h3/htrc_flat_triton.py:214-254, DOT = 0).  Workgroup = one group x SEL_F32_LPW
// leaves, 4 waves; wave w holds the split q - mu of 16 of the group's sampled rows (rows 64 c +
// 16 w .. of row chunk c; rows past the last repeat it, tiles past the last repeat it, as the
// reference pads them, which leaves every maximum unchanged) and the workgroup streams its
// leaves' g rows 16 at a time: each thread fetches its 8 dims of one leaf two blocks ahead into
// registers and splits them once into the block's bf16 terms in LDS (two buffers, one barrier
// per block), which every wave reads as its MFMA operands.
// Products on the bf16 MFMA (16x16x32, rows as A, leaves as B: k-step ks takes lane group grp's
// dims 32 ks + 8 grp .. + 7): g and q - mu each split into bf16 terms that sum to them exactly (a
// bf16 g: one term; TF32 operands: two; fp32: three), every term product formed, so each dim's
// product is exactly the one the fp32 MFMA forms and only the grouping of the fp32 sums differs.
constexpr int SEL_F32_LPW = 1024;  // leaves per workgroup
template <bool QBF, bool SB, bool TF32>
__global__ __launch_bounds__(256) void select_f32_kernel(const void* __restrict__ q, const float* __restrict__ mu,
                                                         int mu_stride, const void* __restrict__ g,
                                                         const float* __restrict__ lz, int64_t nq, int nt, int tile,
                                                         int stride, int group, int g0, int ng,
                                                         const int32_t* __restrict__ perm, int nb, int nb_pad,
                                                         float* __restrict__ sel) {
    constexpr int QB = QBF ? 2 : 4, SBB = SB ? 2 : 4;
    constexpr int NG = SB ? 1 : (TF32 ? 2 : 3), ND = TF32 ? 2 : 3;
    constexpr int RW = SB ? 1 : 2;                             // 16-byte pieces per 8 dims of g
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, col = lane & 15,
              grp = lane >> 4, tid = threadIdx.x;
    const int gi = blockIdx.y, h = blockIdx.z, gg = g0 + gi;
    const int lw0 = blockIdx.x * SEL_F32_LPW, nlw = min(nb - lw0, SEL_F32_LPW);   // leaves [lw0, lw0 + nlw)
    const int nblk = (nlw + 15) / 16;
    const int64_t srow = ((int64_t)h * ng + gi) * nb_pad;
    __shared__ __align__(16) char terms[2][NG][16 * 256];     // block terms: leaf row of 256 B, chunk c at c ^ leaf
    __shared__ float wmax[4][SEL_F32_LPW];                     // per wave: each leaf's max over its rows
    auto split = [&](float (&x)[8], bf16x8 (&t)[3], int n) {
#pragma unroll
        for (int tt = 0; tt < 3; ++tt) {
            if (tt >= n) break;
            const u32x4 u = {pack2bf(x[0], x[1]), pack2bf(x[2], x[3]), pack2bf(x[4], x[5]), pack2bf(x[6], x[7])};
            t[tt] = as_bf16x8(u);
            if (tt + 1 < n) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[2 * e] = __fsub_rn(x[2 * e], __uint_as_float(u[e] << 16));
                    x[2 * e + 1] = __fsub_rn(x[2 * e + 1], __uint_as_float(u[e] & 0xffff0000u));
                }
            }
        }
    };
    // thread tid's part of block b: leaf 16 b + tid / 16 (the last leaf past the range), dims
    // 8 (tid % 16) .. + 7
    auto gfetch = [&](int b, u32x4 (&raw)[RW]) {
        const int leaf = lw0 + min(16 * b + (tid >> 4), nlw - 1);
        const char* p = (const char*)g + ((srow + leaf) * D + 8 * (tid & 15)) * SBB;
#pragma unroll
        for (int u = 0; u < RW; ++u) raw[u] = *(const u32x4*)(p + 16 * u);
    };
    auto gstage = [&](const u32x4 (&raw)[RW], int buf) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if constexpr (SB) x[e] = bf2f((e & 1) ? (raw[0][e >> 1] >> 16) : (raw[0][e >> 1] & 0xffffu));
            else x[e] = TF32 ? tf32_rna(__uint_as_float(raw[e >> 2][e & 3])) : __uint_as_float(raw[e >> 2][e & 3]);
        }
        bf16x8 t[3];
        split(x, t, NG);
        const int lf = tid >> 4, c = tid & 15;
#pragma unroll
        for (int a = 0; a < NG; ++a) *(bf16x8*)(&terms[buf][a][lf * 256 + ((c ^ lf) << 4)]) = t[a];
    };
    for (int i = lane; i < SEL_F32_LPW; i += 64) wmax[w][i] = -INFINITY;
    const float* murow = mu + ((int64_t)h * mu_stride + gg) * D + 8 * grp;
    const int rpt = tile / stride, nsel = group * rpt;
    for (int rc = 0; rc < nsel; rc += 64) {
        const bool active = rc + 16 * w < nsel;                // wave-uniform: the wave has rows here
        bf16x8 dt[4][3];
        if (active) {
            const int j = min(rc + 16 * w + col, nsel - 1);
            const int tt = min(gg * group + j / rpt, nt - 1);
            const int64_t qi = min((int64_t)tt * tile + (j % rpt) * stride, nq - 1);
            const char* qrow = (const char*)q + ((int64_t)h * nq + perm_row(perm, h, nq, qi)) * D * QB;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                float x[8], mx[8];
                load_f32<8, QBF, false>(qrow + (32 * ks + 8 * grp) * QB, x);
                load_f32<8, false, false>(murow + 32 * ks, mx);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[e] = __fsub_rn(x[e], mx[e]);
                    if constexpr (TF32) x[e] = tf32_rna(x[e]);
                }
                split(x, dt[ks], ND);
            }
        }
        // block b: its terms in buffer b % 2; rs holds block b + 1's raw g, refilled with b + 3
        auto step = [&](int b, u32x4 (&rs)[RW]) {
            if (active) {
                const char* tb_ = &terms[b & 1][0][0];
                f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int sum = NG + ND - 2; sum >= 0; --sum)    // smaller products first
#pragma unroll
                    for (int a = 0; a < NG; ++a) {
                        const int bt = sum - a;
                        if (bt < 0 || bt >= ND) continue;
#pragma unroll
                        for (int ks = 0; ks < 4; ++ks) {
                            const bf16x8 gb = *(const bf16x8*)(tb_ + a * (16 * 256) + col * 256 + (((4 * ks + grp) ^ col) << 4));
                            s4 = mfma_bf16(dt[ks][bt], gb, s4);
                        }
                    }
                // rows 4 grp + i of leaf 16 b + col: the max over the wave's 16 rows
                float m = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3]));
                m = grp_max(m);
                if (grp == 0) wmax[w][16 * b + col] = fmaxf(wmax[w][16 * b + col], m);
            }
            if (b + 1 < nblk) gstage(rs, (b + 1) & 1);
            if (b + 3 < nblk) gfetch(b + 3, rs);
            __syncthreads();
        };
        u32x4 ra[RW], rb[RW];
        gfetch(0, ra);
        gstage(ra, 0);
        if (nblk > 1) gfetch(1, ra);
        if (nblk > 2) gfetch(2, rb);
        __syncthreads();
        for (int b = 0; b < nblk; b += 2) {
            step(b, ra);
            if (b + 1 < nblk) step(b + 1, rb);
        }
    }
    for (int i = tid; i < nlw; i += 256) {
        const float m = fmaxf(fmaxf(wmax[0][i], wmax[1][i]), fmaxf(wmax[2][i], wmax[3][i]));
        sel[srow + lw0 + i] = __fadd_rn(m, lz[srow + lw0 + i]);
    }
}

// merge: (h3/htrc_flat_triton.py:257-273) + logZ = mm + log(den).  One workgroup (4 * tile
// threads) per tile.
// Tiles [t0, t0 + gridDim.x) of each head; the partials are the launch's own [H, gridDim.x, ns, tile].
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ pm, const float* __restrict__ pl,
                                                    const float* __restrict__ pacc, int ns, int64_t nq, int t0,
                                                    int tile, const int32_t* __restrict__ perm,
                                                    float* __restrict__ out, float* __restrict__ logz) {
    const int t = t0 + blockIdx.x, h = blockIdx.y;
    const int64_t th = (int64_t)h * gridDim.x + blockIdx.x;   // partial row of the tile
    const int r = threadIdx.x >> 2, part = threadIdx.x & 3;   // 4 threads per row, 32 dims each
    const int64_t qi = (int64_t)t * tile + r;
    if (qi >= nq) return;
    float mm = -INFINITY;
    for (int s = 0; s < ns; ++s) mm = fmaxf(mm, pm[(th * ns + s) * tile + r]);
    if (mm == -INFINITY) mm = 0.0f;
    float den = 0.0f;
    float num[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) num[i] = 0.0f;
    for (int s = 0; s < ns; ++s) {
        const int64_t b = (th * ns + s) * tile + r;
        const float wv = __expf(__fsub_rn(pm[b], mm));
        den = __fadd_rn(den, __fmul_rn(pl[b], wv));
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const f32x4 x = *(const f32x4*)(pacc + b * D + part * 32 + i);
#pragma unroll
            for (int j = 0; j < 4; ++j) num[i + j] = __fadd_rn(num[i + j], __fmul_rn(x[j], wv));
        }
    }
    const float dd = den < 1e-30f ? 1e-30f : den;
    const int64_t orow = (int64_t)h * nq + perm_row(perm, h, nq, qi);
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        f32x4 o = {__fdiv_rn(num[i], dd), __fdiv_rn(num[i + 1], dd), __fdiv_rn(num[i + 2], dd),
                   __fdiv_rn(num[i + 3], dd)};
        *(f32x4*)(out + orow * D + part * 32 + i) = o;
    }
    if (part == 0) logz[orow] = __fadd_rn(mm, __logf(den));
}

// ---------------------------------------------------------------------------------------------
// route: the production path, two launches per layer call.
//   route_select_kernel, one 4-wave workgroup per tile: SEL of every leaf into LDS (bit-exact,
//     the select_kernel arithmetic), top-k -> idx, and each row's largest far-field score;
//   route_kernel, one workgroup per tile: far + near field in one online softmax whose
//     reference max is that score.  NP wave pairs split the keys (large grids: one pair, all
//     keys, five tiles per CU; smaller grids: two or four pairs): pair pr = wave % NP takes
//     its far leaves, then its near tokens, in 32-key blocks, and wave wave / NP of the pair
//     takes half of the tile's rows (32 of 64, or 16 of 32); each block in LDS feeds both.  A
//     pair's blocks stream through a 2-slot LDS ring, loaded one block ahead by direct
//     global->LDS loads split between the two waves; several pairs' partial states merge through
//     LDS, one pair's waves store their rows straight from registers.
// SEL and the partial states never reach HBM.
// ---------------------------------------------------------------------------------------------
template <int RB>
struct RowsN {         // softmax state of the 16 RB rows of one wave
    float m[RB];       // reference max (log2 units), fixed during a pass
    float l[RB];       // this lane's share of the row sums
    f32x4 o[RB][8];    // O^T per row block: dims 16db + 4grp + i of row 16rb + lane%16
};

// p = 2^(u - m) for the log2-domain scores u[rb][0..7] of the RB row blocks (keys
// 16(e/4) + 4grp + e%4 of the block; masked keys -inf), l += p, O^T += V^T P^T.  SHIFTED:
// the scores are u - m already.
template <int RB, bool SHIFTED>
__device__ __forceinline__ void rows_update(RowsN<RB>& st, const float (&sc)[RB][8], const u32x2 (&v)[8][2]) {
    bf16x8 P[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            p[e] = __builtin_amdgcn_exp2f(SHIFTED ? sc[rb][e] : __fsub_rn(sc[rb][e], st.m[rb]));
        st.l[rb] = __fadd_rn(st.l[rb], __fadd_rn(__fadd_rn(__fadd_rn(p[0], p[1]), __fadd_rn(p[2], p[3])),
                                                 __fadd_rn(__fadd_rn(p[4], p[5]), __fadd_rn(p[6], p[7]))));
        P[rb] = to_bf16x8(p);
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        const bf16x8 A = as_bf16x8(v[db][0], v[db][1]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) st.o[rb][db] = mfma_bf16(A, P[rb], st.o[rb][db]);
    }
}

// Ring slot of one 32-key block: [QK A operands 4 KB | PV rows 8 KB | scales 256 B].
constexpr int SLOT_BYTES = 4096 + 8192 + 256;
constexpr int DMA_W0 = 7;                           // loads per block, first wave of a pair
constexpr int DMA_W1 = 6;                           // ... second wave
constexpr int ROUTE_MAX_KX = 8192;                  // near leaves per tile the route kernel holds in LDS
constexpr int64_t ROUTE_MAX_NB = 262144;             // leaves per head (exclusion bits: 32 KB of LDS)
constexpr size_t ROUTE_LDS_MAX = 160 * 1024;         // LDS of one workgroup on gfx950
// Passes of a tile in the route kernels: one at the select launch's reference, and when a row
// total leaves range one more at every row's exact largest score (in range by construction).
constexpr int MAX_PASSES = 2;
// Merge: the wave pairs' partial O, 64 rows x 128 dims each, rows padded to 132 floats.
constexpr int MRG_STRIDE = 132;
// Ring slots per pair: blocks are loaded RS - 1 ahead.  Two slots (one block in flight while the
// other is computed on) measured 1.8% faster than three at cfg3, and their 54 KB leave room for
// a third workgroup per CU, which is slower again (register spills and contention).
constexpr int ROUTE_RS = 2;
// Waves per SIMD the route kernel's register budget allows: three for one wave pair per tile
// (168 VGPRs; the 3 spilled values sit outside the key loops; 3.012 -> 2.995 ms at cfg3), two
// for two pairs (there a 168-VGPR cap spills inside the loops).
template <int NP>
constexpr int route_waves_per_simd() { return NP == 1 ? 3 : 2; }

// The per-(tile, leaf) state is read once per launch by route_select and once by the attend
// kernel's far field.  Non-temporal loads keep such a stream from displacing cached lines
// that others reuse (the K / V rows neighbouring tiles' near fields share).
constexpr bool SEL_NT = false;
constexpr bool FAR_NT = true;

// Per-lane byte offsets of the 32-key block loads (loop invariant): the QK operand chunk of
// lane (col, grp) and the swizzled PV row chunks (see dma_rows).
struct BlockOffsets {
    uint32_t qk[2];                                    // k-steps 0 and 1 (dims 0..63, 64..127)
    uint32_t rows[4];
};

__device__ __forceinline__ BlockOffsets block_offsets(int lane) {
    const int col = lane & 15, grp = lane >> 4, pc = lane & 15;
    BlockOffsets o;
    o.qk[0] = (uint32_t)(col * D + 16 * grp);
    o.qk[1] = o.qk[0] + 64;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 4 * j + grp;                   // rows j*4 + grp, and the same + 16
        o.rows[j] = (uint32_t)(row * 2 * D + 16 * (pc ^ swz(row)));
    }
    return o;
}

// QK operand chunks j (0..3) of lane: [hh = j>>1][ks = j&1][grp][col] <- row (row0[hh] + col),
// bytes (4ks + grp)*16 of an int8 [*, 128] matrix; x0/x1 point at rows row0a/row0b.  One M0.
template <bool NT>
__device__ __forceinline__ void dma_qk(const int8_t* x0, const int8_t* x1, const BlockOffsets& bo, uint32_t slot) {
    dma_x4<NT>(sbase(x0), bo.qk[0], sbase(x0, 1024), bo.qk[1], sbase(x1, 2048), bo.qk[0], sbase(x1, 3072), bo.qk[1], slot);
}

// PV rows of a 32-key block: ring chunk s = 64j + lane (j = 0..7) holds the 16-byte chunk
// (s % 16) ^ swz(row) of row s / 16 (rows 0..15 from x0, 16..31 from x1) of a bf16 [*, 128]
// matrix; swz(row) = swz(row - 16), so both halves share the lane offsets.  Chunks 0, 1:
template <bool NT>
__device__ __forceinline__ void dma_rows01(const uint16_t* x0, const BlockOffsets& bo, uint32_t slot) {
    dma_x2<NT>(sbase(x0), bo.rows[0], sbase(x0, 1024), bo.rows[1], slot + 4096);
}
// chunks 2..7:
template <bool NT>
__device__ __forceinline__ void dma_rows27(const uint16_t* x0, const uint16_t* x1, const BlockOffsets& bo,
                                           uint32_t slot) {
    dma_x2<NT>(sbase(x0), bo.rows[2], sbase(x0, 1024), bo.rows[3], slot + 4096 + 2048);
    dma_x4<NT>(sbase(x1), bo.rows[0], sbase(x1, 1024), bo.rows[1], sbase(x1, 2048), bo.rows[2], sbase(x1, 3072),
           bo.rows[3], slot + 8192);
}

// route_select: first launch of the fused production path, one workgroup (4 waves) per tile.
//   SEL of every leaf (bit-exact, the select_kernel arithmetic) into LDS, its kx largest
//   (idx ascending, leaves < sink forced in), and per row the largest far-field score, the
//   fixed softmax reference of route_kernel (the tile maximum when rows are sampled).
// Small register and LDS footprint: several tiles share a CU, so their load latency and their
// top-k overlap.  SEL never reaches HBM.
// MULTI: tile groups of G > 1 tiles (keys merged by max over the tiles); NRB = tile / 16 row
// blocks of 16 rows per tile.
// GK: the top-k keys of the tile group sit in global memory (keys_ws [H, ng, nb_pad]) instead of
// LDS, for rows of more leaves than the LDS holds.  The launch covers tile groups
// [g0, g0 + ng) of each head; the state rows and idx are the launch's own ([H, ng, ...]).
constexpr int SEL_RING = 3;                         // route_select ring slots per wave
constexpr int ROUTE_NB_LDS = 16384;                 // leaves per head whose keys route_select keeps in LDS
template <bool MULTI, int NRB, bool GK>
__global__ __launch_bounds__(256, 4) void route_select_kernel(
    const int8_t* __restrict__ dq8, const float* __restrict__ sdq, const int8_t* __restrict__ g8,
    const float* __restrict__ sg, const float* __restrict__ lz, int nt, int group, int g0, int ng, int nb,
    int nb_pad, int kx, int sink, int stride, int32_t* __restrict__ idx, float* __restrict__ rowmax,
    uint32_t* __restrict__ keys_ws) {
    extern __shared__ uint32_t keys_lds[];    // [nb] unless GK
    __shared__ TopkSmem sm;
    __shared__ float red_m[4][64];
    // each wave's own ring of 16-leaf groups: g8 rows as the two 1 KB QK operand chunks
    // (kss = 0, 1; lane-linear), then sg (64 B) and lz (64 B)
    constexpr int SEL_SLOT = 2048 + 128;
    __shared__ __align__(16) char sring[4][SEL_RING][SEL_SLOT];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // one workgroup per tile group (G tiles sharing a centre, state and near leaves; G = 1: a tile)
    const uint32_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int gi = (int)(blk % (uint32_t)ng), h = (int)(blk / (uint32_t)ng);
    const int64_t gs = (int64_t)h * ng + gi;   // state / idx row (the launch's window)
    uint32_t* keys = GK ? keys_ws + gs * nb_pad : keys_lds;
    constexpr int TR = 16 * NRB;              // rows per tile
    const int ts = TR / stride;
    struct SelOps {
        i32x4 a[2];
        f32x4 sg, lz;
    };
    const uint32_t ring_lds = lds_addr(&sring[w][0][0]);
    const uint32_t voff0 = (uint32_t)(col * D + 16 * grp), voff1 = voff0 + 64;
    // group gj of this wave (leaves c = 16 w + 64 gj ..) into ring slot gj % SEL_RING: three
    // direct loads; lane (col, grp) of operand chunk kss gets bytes 64 kss + 16 grp of row col
    auto sel_issue = [&](int gj, int ngr) {
        if (gj >= ngr) return;
        const int64_t s0 = gs * nb_pad + 16 * w + 64 * gj;
        const uint32_t slot = ring_lds + (uint32_t)(gj % SEL_RING) * SEL_SLOT;
        dma16s<SEL_NT>(g8 + s0 * D, voff0, slot);
        dma16s<SEL_NT>(g8 + s0 * D, voff1, slot + 1024);
        if (lane < 8) dma16<SEL_NT>(lane < 4 ? sg + s0 + 4 * lane : lz + s0 + 4 * (lane - 4), slot + 2048);
    };
    auto sel_read = [&](SelOps& o, int gj) {
        const char* slot = &sring[w][gj % SEL_RING][0];
#pragma unroll
        for (int kss = 0; kss < 2; ++kss) o.a[kss] = *(const i32x4*)(slot + 1024 * kss + 16 * lane);
        o.sg = *(const f32x4*)(slot + 2048 + 16 * grp);
        o.lz = *(const f32x4*)(slot + 2048 + 64 + 16 * grp);
    };
    i32x4 b[NRB][2];
    bool val[NRB];
    float srow[NRB];
    float rmax[NRB];                          // row max of the far scores
    bool first = true;                        // first tile of the group: set the keys, later: max
    auto sel_block = [&](const SelOps& o, int c) {
        i32x4 acc[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            acc[rb] = mfma_i8(o.a[0], b[rb][0], i32x4{0, 0, 0, 0});
            acc[rb] = mfma_i8(o.a[1], b[rb][1], acc[rb]);
        }
        // No masks: rows past the sampled ones repeat row 0 (the maximum is unchanged; their
        // rmax is never written), and leaves past nb have lz = -inf (sg = 0) in the state.
        float best[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            best[i] = -INFINITY;
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) {
                const float x = __fmul_rn((float)acc[rb][i], __fmul_rn(srow[rb], o.sg[i]));
                best[i] = fmaxf(best[i], x);
                rmax[rb] = fmaxf(rmax[rb], __fadd_rn(x, o.lz[i]));
            }
            best[i] = col_max(best[i]);
        }
        if (col == 0) {               // leaf l is always this lane's: no race across tiles
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int l = c + 4 * grp + i;
                if (l < nb) {
                    const uint32_t key = l < sink ? 0xffffffffu : order_key(__fadd_rn(best[i], o.lz[i]));
                    keys[l] = (!MULTI || first) ? key : max(keys[l], key);
                }
            }
        }
    };
    for (int j = 0; j < (MULTI ? group : 1); ++j) {
        const int t = (g0 + gi) * group + j;
        if (t >= nt) break;                   // padded tiles repeat the last one
        const int64_t th = (int64_t)h * nt + t;
        load_rows_i8(dq8, th * TR, stride, ts, col, grp, b, val);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            srow[rb] = sdq[th * TR + (int64_t)(val[rb] ? 16 * rb + col : 0) * stride];
            rmax[rb] = -INFINITY;
            // consumed before the first direct load: the compiler's own wait for them would
            // otherwise drain the ring
            asm volatile("" : : "v"(b[rb][0]), "v"(b[rb][1]), "v"(srow[rb]));
        }
        // wave w: 16-leaf groups c = 16 w + 64 gj through its ring, loaded SEL_RING - 1 ahead
        const int ngr = 16 * w < nb ? (nb - 16 * w + 63) / 64 : 0;
#pragma unroll
        for (int gj = 0; gj < SEL_RING - 1; ++gj) sel_issue(gj, ngr);
        for (int gj = 0; gj < ngr; ++gj) {
            if (gj + SEL_RING - 2 < ngr) wait_vmcnt<3 * (SEL_RING - 2)>();   // the later groups stay in flight
            else wait_vmcnt<0>();
            SelOps o;
            sel_read(o, gj);
            sel_issue(gj + SEL_RING - 1, ngr);       // into the slot of group gj - 1, read last iteration
            sel_block(o, 16 * w + 64 * gj);
        }
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {    // row r = stride * (16 rb + col) of the sampled rows
            const float mx = grp_max(rmax[rb]);
            if (grp == 0) red_m[w][16 * rb + col] = mx;
        }
        __syncthreads();
        if (w == 0) {
            const int r = lane;
            float m = r < ts ? fmaxf(fmaxf(red_m[0][r], red_m[1][r]), fmaxf(red_m[2][r], red_m[3][r])) : -INFINITY;
            if (stride != 1) m = wave_max(m); // sampled rows: one reference for the whole tile
            if (r < TR) rowmax[th * TR + r] = m;
        }
        if (MULTI) __syncthreads();           // red_m is free for the next tile
        first = false;
    }
    const int kxe = min(kx, nb);
    if (kxe > 0) topk_row([&](int l) { return keys[l]; }, nb, kxe, sm, idx + gs * kxe, nullptr, nullptr);
}

// Largest scores of a wave's rows: the repair of a missed softmax reference in the route kernels.
template <int RB>
struct RowMax {
    float m[RB];
};

// The largest score (log2 units) of each of this wave's rows (rowb + 16 rb + col, rowb wave-uniform,
// lane (col, grp)) over
// a key part of route_kernel: the far leaves [lo, hi) not excluded, then the near tokens
// [e_lo, e_hi) of the list sidx, 16 keys per MFMA pair with both operands loaded straight from
// global memory; every lane of a row's column ends with it.  It runs only when a tile's
// reference missed.  Every lane-dependent address is derived from a lane index redefined through
// an empty asm here, so the compiler cannot hoist them out of the caller's pass loop (they would
// stay live, and spill, through its key loops).
template <int LEAF, int RB>
__device__ __forceinline__ RowMax<RB> route_exact_max(const int8_t* dq8, const float* sdq, const int8_t* q8,
                                                   const float* sq, float scale, const int8_t* g8, const float* sg,
                                                   const float* lz, const uint32_t* exbits, int64_t srow0, int lo,
                                                   int hi, const int8_t* k8, const float* ks, const uint32_t* sidx,
                                                   int64_t kh, int e_lo, int e_hi, int64_t rowb) {
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const int col = lane & 15, grp = lane >> 4;
    const int64_t row0 = rowb + col;
    RowMax<RB> mx;
    i32x4 bq[RB][2];
    float srow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int64_t p = row0 + 16 * rb;
        bq[rb][0] = *(const i32x4*)(dq8 + p * D + 16 * grp);
        bq[rb][1] = *(const i32x4*)(dq8 + p * D + 64 + 16 * grp);
        srow[rb] = __fmul_rn(sdq[p], LOG2E);
        mx.m[rb] = -INFINITY;
    }
    for (int c = lo; c < hi; c += 16) {           // rows < nb_pad; leaves >= nb are excluded
        const int64_t r = srow0 + c;
        const i32x4 A0 = *(const i32x4*)(g8 + (r + col) * D + 16 * grp);
        const i32x4 A1 = *(const i32x4*)(g8 + (r + col) * D + 64 + 16 * grp);
        const f32x4 sgv = *(const f32x4*)(sg + r + 4 * grp), lzv = *(const f32x4*)(lz + r + 4 * grp);
        const uint32_t exw = exbits[c >> 5] >> ((c & 31) + 4 * grp);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const i32x4 acc = mfma_i8(A1, bq[rb][1], mfma_i8(A0, bq[rb][0], i32x4{0, 0, 0, 0}));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lzm = (exw >> i) & 1u ? -INFINITY : lzv[i];
                mx.m[rb] = fmaxf(mx.m[rb], __fmaf_rn((float)acc[i], __fmul_rn(srow[rb], sgv[i]), __fmul_rn(lzm, LOG2E)));
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int64_t p = row0 + 16 * rb;
        bq[rb][0] = *(const i32x4*)(q8 + p * D + 16 * grp);
        bq[rb][1] = *(const i32x4*)(q8 + p * D + 64 + 16 * grp);
        srow[rb] = __fmul_rn(__fmul_rn(sq[p], scale), LOG2E);
    }
    for (int j = e_lo; j < e_hi; j += 16) {       // 16-token runs of the near leaves
        const int64_t tok = kh + (int64_t)__builtin_amdgcn_readfirstlane(sidx[j / LEAF]) * LEAF + (j % LEAF);
        const i32x4 A0 = *(const i32x4*)(k8 + (tok + col) * D + 16 * grp);
        const i32x4 A1 = *(const i32x4*)(k8 + (tok + col) * D + 64 + 16 * grp);
        const f32x4 ksv = *(const f32x4*)(ks + tok + 4 * grp);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const i32x4 acc = mfma_i8(A1, bq[rb][1], mfma_i8(A0, bq[rb][0], i32x4{0, 0, 0, 0}));
#pragma unroll
            for (int i = 0; i < 4; ++i) mx.m[rb] = fmaxf(mx.m[rb], __fmul_rn((float)acc[i], __fmul_rn(srow[rb], ksv[i])));
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) mx.m[rb] = grp_max(mx.m[rb]);
    return mx;
}

// RB = tile / 32: 16-row blocks per wave (tiles of 64 or 32 rows); NP wave pairs split the keys;
// RS ring slots per pair.
template <int LEAF, int RB, int NP, int RS>
__global__ __launch_bounds__(128 * NP, route_waves_per_simd<NP>()) void route_kernel(
    const int8_t* __restrict__ q8, const float* __restrict__ sq, const int8_t* __restrict__ dq8,
    const float* __restrict__ sdq, const int8_t* __restrict__ g8, const float* __restrict__ sg,
    const float* __restrict__ lz, const uint16_t* __restrict__ vb, const int8_t* __restrict__ k8,
    const float* __restrict__ ks, const uint16_t* __restrict__ v, const int32_t* __restrict__ idx,
    const float* __restrict__ rowmax, int64_t nq, int nt, int group, int g0, int ng, const int32_t* __restrict__ perm,
    int64_t nk, int nb, int nb_pad, int kxe, float scale, float* __restrict__ out, float* __restrict__ logz) {
    constexpr int NT = 128 * NP;                               // threads
    __shared__ __align__(16) char ring[NP][RS][SLOT_BYTES];    // one per wave pair; also merge staging
    // sized by the launch: exclusion bits [nb / 32 + 1], then the tile's near leaves [kxe], so
    // small shapes leave room for more tiles per CU
    extern __shared__ __align__(16) uint32_t route_dyn[];
    uint32_t* exbits = route_dyn;
    uint32_t* sidx = route_dyn + (nb / 32 + 1);
    __shared__ float red_m[64], red_l[NP][64];
    __shared__ int redo;
    constexpr int TR = 32 * RB;                                // rows per tile
    // merge staging in the ring: all rows at once, or one row half (one wave of each pair) at a time
    constexpr bool MRG2 = NP * TR * MRG_STRIDE * 4 > NP * RS * SLOT_BYTES;
    constexpr int RR = MRG2 ? TR / 2 : TR;                     // rows per merge round
    static_assert(NP * RR * MRG_STRIDE * 4 <= NP * RS * SLOT_BYTES, "merge staging");
    float* mrg = (float*)&ring[0][0][0];                       // merge staging: NP x 64 x MRG_STRIDE floats
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar bookkeeping
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const int pr = wv % NP, hr = wv / NP;                      // key part (wave pair), row half
    auto row_total = [&](int r) {                              // a row's sum over the NP parts
        if constexpr (NP == 4)
            return __fadd_rn(__fadd_rn(red_l[0][r], red_l[1][r]), __fadd_rn(red_l[2][r], red_l[3][r]));
        else if constexpr (NP == 2)
            return __fadd_rn(red_l[0][r], red_l[1][r]);
        else
            return red_l[0][r];
    };
    // 1-D grid over (tile, head), tile fastest: each XCD runs a contiguous run of tiles of one
    // head at a time, so the near-field leaves adjacent tiles share are fetched into one L2.
    // The launch covers the tiles of groups [g0, g0 + ng) of each head; state and idx rows are the
    // launch's own.
    const int tb = g0 * group, ntw = min(nt, (g0 + ng) * group) - tb;
    const uint32_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int t = tb + (int)(blk % (uint32_t)ntw), h = (int)(blk / (uint32_t)ntw);
    const int64_t th = (int64_t)h * nt + t;
    const int64_t gs = (int64_t)h * ng + (t / group - g0);    // state / routing row: the tile's group
    const int64_t kh = (int64_t)h * nk;
    const int64_t row0 = th * TR + 16 * RB * hr + col;         // this lane's rows: row0 (+ 16 when RB = 2)
    // ---- routing of this tile (route_select_kernel)
    // exclusion bits: the selected (near) leaves, and every leaf >= nb, so the far loop needs no
    // range test (far blocks are 32-leaf aligned and a pair's range ends on a 32-leaf boundary
    // or at nb)
    for (int i = threadIdx.x; i <= nb / 32; i += NT) {
        const int past = nb - 32 * i;          // leaves of word i below nb
        exbits[i] = past >= 32 ? 0u : (past <= 0 ? ~0u : ~0u << past);
    }
    for (int j = threadIdx.x; j < kxe; j += NT) sidx[j] = (uint32_t)idx[gs * kxe + j];
    float mref[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float m = rowmax[row0 + 16 * rb];
        mref[rb] = m == -INFINITY ? 0.0f : __fmul_rn(m, LOG2E);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < kxe; j += NT) atomicOr(&exbits[sidx[j] >> 5], 1u << (sidx[j] & 31));
    // ---- key ranges: pair q owns far leaves [q lpw, q lpw + lpw) and near list positions
    // [q epw, q epw + epw), in 32-key blocks; every wave runs the longest pair's step count
    const int lpw = ((nb + NP - 1) / NP + 31) / 32 * 32;
    const int e_n = kxe * LEAF;
    const int epw = ((e_n + NP - 1) / NP + 31) / 32 * 32;
    const int lo = pr * lpw, hi = min(nb, lo + lpw);
    const int e_lo = pr * epw, e_hi = min(e_n, e_lo + epw);
    const int nf = hi > lo ? (hi - lo + 31) / 32 : 0;
    const int nn = e_hi > e_lo ? (e_hi - e_lo + 31) / 32 : 0;
    const int sf_steps = min(nb, lpw) > 0 ? (min(nb, lpw) + 31) / 32 : 0;        // pair 0 is the longest
    const int sn_steps = min(e_n, epw) > 0 ? (min(e_n, epw) + 31) / 32 : 0;
    // far steps rounded up to even (an odd count takes one empty step), so the near blocks
    // start in ring slot 0 and the last far step issues the first of them
    const int sf_even = (sf_steps + 1) & ~1;
    const int64_t srow0 = gs * nb_pad;
    char* pring = &ring[pr][0][0];
    const uint32_t pring_lds = lds_addr(pring);
    auto wait_block = [&](int bi, int nblk) {    // this wave's loads of block bi have landed
        if (RS == 3 && bi + 1 < nblk) {             // block bi + 1 may still be in flight
            if (hr == 0) wait_vmcnt<DMA_W0>();
            else wait_vmcnt<DMA_W1>();
        } else {
            wait_vmcnt<0>();
        }
    };
    const BlockOffsets bo = block_offsets(lane);
    // This wave's share of the loads of a 32-key block with rows r0.. and r1.. (16 each).  The
    // scale area gets 32 floats from s_lo (lanes 0..7) and 32 from s_hi (lanes 8..15); a near
    // block's runs hold only 16 tokens each, so there (nlim = 3) lanes 4..7 and 12..15 repeat
    // the run's first 16 scales instead of reading past it.
    auto load_block = [&](auto nt_, uint32_t slot, const int8_t* X8, const uint16_t* XV, int64_t r0, int64_t r1,
                          const float* s_lo, const float* s_hi, int nlim) {
        constexpr bool NTL = decltype(nt_)::value;
        if (hr == 0) {
            dma_qk<NTL>(X8 + r0 * D, X8 + r1 * D, bo, slot);
            dma_rows01<NTL>(XV + r0 * D, bo, slot);
            // (the saddr form, one base per lane half: no 64-bit lane address held across the loop)
            if (lane < 8) dma16s<NTL>(s_lo, (uint32_t)(16 * (lane & nlim)), slot + 12288);
            else if (lane < 16) dma16s<NTL>(s_hi, (uint32_t)(16 * (lane & nlim)), slot + 12288);
        } else {
            dma_rows27<NTL>(XV + r0 * D, XV + r1 * D, bo, slot);
        }
    };
    // near block bi (list positions e_lo + 32 bi, + 16): the 16-token runs start there (past
    // e_hi: the range start again, loaded and masked); token = leaf * LEAF + position % LEAF
    auto run_pos = [&](int j) { return j < e_hi ? j : e_lo; };
    auto issue_near = [&](int bi, int slot) {
        if (bi >= nn) return;
        const int e0 = e_lo + 32 * bi, ja = run_pos(e0), jb = run_pos(e0 + 16);
        const int64_t r0 = kh + (int64_t)__builtin_amdgcn_readfirstlane(sidx[ja / LEAF]) * LEAF + (ja % LEAF);
        const int64_t r1 = kh + (int64_t)__builtin_amdgcn_readfirstlane(sidx[jb / LEAF]) * LEAF + (jb % LEAF);
        load_block(std::false_type{}, pring_lds + slot * SLOT_BYTES, k8, v, r0, r1, ks + r0, ks + r1, 3);
    };
    static_assert(RS == 2, "the far / near block stream alternates two ring slots");
    // LDS addresses of this lane's PV operand reads (slot 0, keys 0..15 of a block): the slot's
    // and the second key half's offsets are immediates of the reads
    uint32_t tra[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        tra[db] = pring_lds + 4096 + tr_offset(0, db, lane);
        asm volatile("" : "+v"(tra[db]));   // one register each: no add at every read
    }
    RowsN<RB> st;
#pragma unroll 1
    for (int pass = 0; pass < MAX_PASSES; ++pass) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            st.m[rb] = mref[rb];
            st.l[rb] = 0.0f;
#pragma unroll
            for (int db = 0; db < 8; ++db) st.o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        {   // ---- far field: S^T = g8 dq8^T, score = dot * sdq * sg + lz, excluded leaves masked
            i32x4 bq[RB][2];
            float srow[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int64_t p = row0 + 16 * rb;
                bq[rb][0] = *(const i32x4*)(dq8 + p * D + 16 * grp);
                bq[rb][1] = *(const i32x4*)(dq8 + p * D + 64 + 16 * grp);
                srow[rb] = __fmul_rn(sdq[p], LOG2E);
                // loaded before the first DMA: the compiler's own wait for them would drain the ring
                asm volatile("" : : "v"(bq[rb][0]), "v"(bq[rb][1]), "v"(srow[rb]), "v"(mref[rb]));
            }
            __syncthreads();            // exbits complete; the ring is free (merge / earlier pass)
            auto issue = [&](int bi, int slot) {
                if (bi >= sf_even) {    // past the far steps: the near field's first block
                    issue_near(bi - sf_even, slot);
                    return;
                }
                if (bi >= nf) return;
                const int64_t r0 = srow0 + lo + 32 * bi;
                load_block(std::integral_constant<bool, FAR_NT>{}, pring_lds + slot * SLOT_BYTES, g8, vb, r0, r0 + 16,
                           sg + r0, lz + r0, 7);
            };
            // one step per 32-leaf block; the ring slot of block bi is bi % RS, a constant in each
            // of the RS unrolled steps, so every LDS read uses an immediate offset
            auto step = [&](auto S_, int bi) {
                constexpr int S = decltype(S_)::value;
                if (bi < nf) wait_block(bi, nf);
                __syncthreads();        // the partner's loads have landed too; slot (bi - 1) % RS is free
                issue(bi + RS - 1, (S + RS - 1) % RS);
                if (bi >= nf) return;
                const char* slot = pring + S * SLOT_BYTES;
                const int c0 = lo + 32 * bi;
                const uint32_t exw = exbits[c0 >> 5] >> (4 * grp);       // bit 16 hh + i: this lane's key
                float sc[RB][8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const i32x4 A0 = *(const i32x4*)(slot + ((hh * 2 + 0) * 64 + lane) * 16);
                    const i32x4 A1 = *(const i32x4*)(slot + ((hh * 2 + 1) * 64 + lane) * 16);
                    i32x4 acc[RB];
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        acc[rb] = mfma_i8(A0, bq[rb][0], i32x4{0, 0, 0, 0});
                        acc[rb] = mfma_i8(A1, bq[rb][1], acc[rb]);
                    }
                    const f32x4 sgv = *(const f32x4*)(slot + 12288 + (16 * hh + 4 * grp) * 4);
                    const f32x4 lzv = *(const f32x4*)(slot + 12288 + 128 + (16 * hh + 4 * grp) * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // excluded key: lz -> -inf, one bit select (v_bfi_b32) on the sign-extended bit
                        const uint32_t ex = (uint32_t)__builtin_amdgcn_sbfe((int)exw, 16 * hh + i, 1);
                        uint32_t lzb;
                        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(lzb) : "v"(ex), "v"(0xff800000u), "v"(__float_as_uint(lzv[i])));
                        const float lzm = __uint_as_float(lzb);
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb)   // score - m: the bias lz log2e - m in one rounding
                            sc[rb][4 * hh + i] = fmaf((float)acc[rb][i], __fmul_rn(srow[rb], sgv[i]),
                                                      __fmaf_rn(lzm, LOG2E, -st.m[rb]));
                    }
                }
                u32x2 pvop[8][2];
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) pvop[db][hf] = tr_read(tra[db] + S * SLOT_BYTES + 4096 * hf);
                rows_update<RB, true>(st, sc, pvop);
            };
            issue(0, 0);
#pragma unroll 1
            for (int bi = 0; bi < sf_even; bi += 2) {
                step(std::integral_constant<int, 0>{}, bi);
                step(std::integral_constant<int, 1>{}, bi + 1);
            }
        }
        {   // ---- near field: S^T = k8 q8^T, score = dot * sq * ks * scale
            i32x4 bq[RB][2];
            float srow[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int64_t p = row0 + 16 * rb;
                bq[rb][0] = *(const i32x4*)(q8 + p * D + 16 * grp);
                bq[rb][1] = *(const i32x4*)(q8 + p * D + 64 + 16 * grp);
                srow[rb] = __fmul_rn(__fmul_rn(sq[p], scale), LOG2E);
                asm volatile("" : : "v"(bq[rb][0]), "v"(bq[rb][1]), "v"(srow[rb]));
            }
            // the near blocks continue the far stream: block 0 was issued by the last far step,
            // into slot 0; every wave is done with the far blocks once it passes the first near
            // step's barrier
            auto issue = [&](int bi, int slot, uint32_t la, uint32_t lb) {
                if (bi >= nn) return;
                const int e0 = e_lo + 32 * bi, ja = run_pos(e0), jb = run_pos(e0 + 16);
                const int64_t r0 = kh + (int64_t)__builtin_amdgcn_readfirstlane(la) * LEAF + (ja % LEAF);
                const int64_t r1 = kh + (int64_t)__builtin_amdgcn_readfirstlane(lb) * LEAF + (jb % LEAF);
                load_block(std::false_type{}, pring_lds + slot * SLOT_BYTES, k8, v, r0, r1, ks + r0, ks + r1, 3);
            };
            auto step = [&](auto S_, int bi) {
                constexpr int S = decltype(S_)::value;
                // leaves of block bi + RS - 1, read before the waits so their LDS latency is hidden
                const int en = e_lo + 32 * (bi + RS - 1);
                const uint32_t la = sidx[run_pos(en) / LEAF], lb = sidx[run_pos(en + 16) / LEAF];
                if (bi < nn) wait_block(bi, nn);
                __syncthreads();
                issue(bi + RS - 1, (S + RS - 1) % RS, la, lb);
                if (bi >= nn) return;
                const char* slot = pring + S * SLOT_BYTES;
                const int e0 = e_lo + 32 * bi;
                float sc[RB][8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const i32x4 A0 = *(const i32x4*)(slot + ((hh * 2 + 0) * 64 + lane) * 16);
                    const i32x4 A1 = *(const i32x4*)(slot + ((hh * 2 + 1) * 64 + lane) * 16);
                    i32x4 acc[RB];
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        acc[rb] = mfma_i8(A0, bq[rb][0], i32x4{0, 0, 0, 0});
                        acc[rb] = mfma_i8(A1, bq[rb][1], acc[rb]);
                    }
                    // ks of the 32 tokens: run 0 at bytes 0..63, run 1 at 128..191
                    const f32x4 ksv = *(const f32x4*)(slot + 12288 + 128 * hh + 16 * grp);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // score - m in one rounding
                        if constexpr (LEAF % 32 == 0) {   // the near list is whole 32-token blocks
#pragma unroll
                            for (int rb = 0; rb < RB; ++rb)
                                sc[rb][4 * hh + i] = __fmaf_rn((float)acc[rb][i], __fmul_rn(srow[rb], ksv[i]), -st.m[rb]);
                        } else {                          // leaf 16: the last block may be half empty
                            const bool ok = (e0 + 16 * hh + 4 * grp + i) < e_hi;
#pragma unroll
                            for (int rb = 0; rb < RB; ++rb)
                                sc[rb][4 * hh + i] = __fmaf_rn((float)acc[rb][i], __fmul_rn(srow[rb], ksv[i]),
                                                               ok ? -st.m[rb] : -INFINITY);
                        }
                    }
                }
                u32x2 pvop[8][2];
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) pvop[db][hf] = tr_read(tra[db] + S * SLOT_BYTES + 4096 * hf);
                rows_update<RB, true>(st, sc, pvop);
            };
#pragma unroll 1
            for (int bi = 0; bi < sn_steps; bi += 2) {
                step(std::integral_constant<int, 0>{}, bi);
                if (bi + 1 < sn_steps) step(std::integral_constant<int, 1>{}, bi + 1);
            }
        }
        // Row totals over the NP key parts (all at the same reference).  A total outside
        // [2^-60, 2^64] means the reference missed the row's maximum by more than 60 octaves
        // (an outlier key far above the far-field maximum, or rows under a sampled tile
        // reference far below it; never observed on real scores): the tile is redone once at
        // every row's exact largest score, where each row total lies in [1, keys].
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float lt = grp_sum(st.l[rb]);
            if (grp == 0) red_l[pr][16 * RB * hr + 16 * rb + col] = lt;
        }
        if (threadIdx.x == 0) redo = 0;
        __syncthreads();
        bool bad = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float tot = row_total(16 * RB * hr + 16 * rb + col);
            if (!(tot >= 0x1p-60f && tot <= 0x1p64f)) bad = true;
        }
        if (bad) redo = 1;
        __syncthreads();
        if (__builtin_expect(redo == 0 || pass + 1 == MAX_PASSES, 1)) break;
        const RowMax<RB> mx = route_exact_max<LEAF, RB>(dq8, sdq, q8, sq, scale, g8, sg, lz, exbits, srow0, lo, hi, k8,
                                                        ks, sidx, kh, e_lo, e_hi, th * TR + 16 * RB * hr);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
            if (grp == 0) red_l[pr][16 * RB * hr + 16 * rb + col] = mx.m[rb];
        __syncthreads();
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = 16 * RB * hr + 16 * rb + col;
            float m = red_l[0][r];
#pragma unroll
            for (int s = 1; s < NP; ++s) m = fmaxf(m, red_l[s][r]);
            if (m > -INFINITY) mref[rb] = m;
        }
    }
    if constexpr (NP == 1) {
        // one pair: each wave holds its rows' finished O^T; lanes (col, grp) write dims
        // 16 db + 4 grp .. + 3 of row 16 RB hr + 16 rb + col, normalised by the row total
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = 16 * RB * hr + 16 * rb + col;
            const float den = red_l[0][r];
            const float inv = 1.0f / (den < 1e-30f ? 1e-30f : den);
            const int64_t qi = (int64_t)t * TR + r;
            if (qi < nq) {
                const int64_t orow = (int64_t)h * nq + perm_row(perm, h, nq, qi);
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                    const f32x4 o = st.o[rb][db];
                    *(f32x4*)(out + orow * D + 16 * db + 4 * grp) =
                        f32x4{__fmul_rn(o[0], inv), __fmul_rn(o[1], inv), __fmul_rn(o[2], inv), __fmul_rn(o[3], inv)};
                }
                if (grp == 0) logz[orow] = __fadd_rn(__fmul_rn(st.m[rb], LN2), __logf(den));   // m in log2 units
            }
        }
        return;
    }
    // ---- merge: every pair used the same reference per row, so the partial sums simply add
    // (h3/htrc_flat_triton.py:263-273 with equal maxima).  MRG2: two rounds, the rows of row
    // half 0, then of row half 1, so the staging fits a 2-slot ring.
#pragma unroll
    for (int round = 0; round < (MRG2 ? 2 : 1); ++round) {
        if (!MRG2 || hr == round) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int r = 16 * RB * hr + 16 * rb + col;
                if (pr == 0 && grp == 0) red_m[r] = st.m[rb];
                float* dst = mrg + (pr * RR + r - round * RR) * MRG_STRIDE + 4 * grp;
#pragma unroll
                for (int db = 0; db < 8; ++db) *(f32x4*)(dst + 16 * db) = st.o[rb][db];
            }
        }
        __syncthreads();
        constexpr int TPR = NT / RR, DPT = D / TPR;                // threads per row, dims per thread
        const int r_loc = threadIdx.x / TPR, part = threadIdx.x % TPR, r_out = round * RR + r_loc;
        const float den = row_total(r_out);
        const float inv = 1.0f / (den < 1e-30f ? 1e-30f : den);
        const int64_t qi = (int64_t)t * TR + r_out;
        if (qi < nq) {
            const int64_t orow = (int64_t)h * nq + perm_row(perm, h, nq, qi);
#pragma unroll
            for (int u = 0; u < DPT / 4; ++u) {
                const int dl = DPT * part + 4 * u;
                f32x4 acc = *(const f32x4*)(mrg + r_loc * MRG_STRIDE + dl);
#pragma unroll
                for (int s = 1; s < NP; ++s) {
                    const f32x4 y = *(const f32x4*)(mrg + (s * RR + r_loc) * MRG_STRIDE + dl);
                    acc = f32x4{__fadd_rn(acc[0], y[0]), __fadd_rn(acc[1], y[1]), __fadd_rn(acc[2], y[2]),
                                __fadd_rn(acc[3], y[3])};
                }
                *(f32x4*)(out + orow * D + dl) = f32x4{__fmul_rn(acc[0], inv), __fmul_rn(acc[1], inv),
                                                       __fmul_rn(acc[2], inv), __fmul_rn(acc[3], inv)};
            }
            if (part == 0) logz[orow] = __fadd_rn(__fmul_rn(red_m[r_out], LN2), __logf(den));   // m in log2 units
        }
        if (MRG2 && round == 0) __syncthreads();                   // the staging is reused
    }
}

// ---------------------------------------------------------------------------------------------
// route16: the fused production path for the 16-bit state stores (store="fp8": e4m3 g / vb with
// row scales; store="bf16"), two launches per tile window like route:
//   route_select16_kernel, one 4-wave workgroup per tile group: SEL of every leaf with the
//     arithmetic of select16_kernel (bit-exact), kept in LDS, its kx largest (leaves < sink
//     forced in) and every row's largest far-field score, the fixed softmax reference;
//   route16_kernel, one workgroup of two waves per tile (each wave 16 RB rows: 32 at tile 64,
//     so every LDS operand read feeds two row blocks): one continuous stream of 32-key blocks,
//     the far leaves first, then the near tokens, each block staged once in LDS for both waves
//     through a 2-slot ring, the next block's loads issued before the current block is
//     computed.  Every block arrives by direct global->LDS loads (each wave its 16 rows); fp8
//     far blocks stay e4m3 codes in LDS, widened to fp16 (value * 2^-8, exactly) as the operands
//     are read.  Far: score = (dq . g) (* 256 sg) + lz, PV with
//     fp16(p * 256 sv) . vb (fp8) or bf16(p) . vb (bf16); near: score = (q . k) * scale (bf16),
//     PV bf16(p) . v -- the products of tile16_kernel, in one softmax whose reference is the
//     row's far-field maximum (redone with a moved reference if a row total leaves
//     [2^-60, 2^64], as route_kernel).
// ---------------------------------------------------------------------------------------------
// 16-byte position of chunk c of row r of 128-byte rows (e4m3 codes) staged in LDS: c ^ sw8(r).
// A read of 8 bytes per lane whose 32 lanes touch 16 rows, rows 16 h + 0..15 or 4 g + 0..3,
// 16 + 4 g + 0..3 (g = 2 p, 2 p + 1), covers all 64 banks once: sw8 maps each such set of rows
// one-to-one onto (r % 2, position), while r & 7 would put rows r, r + 8 (resp. r + 16) on the
// same banks.
__device__ __forceinline__ int sw8(int r) { return ((r >> 1) & 7) ^ ((r >> 2) & 4); }

template <bool FP8, int NRB>
__global__ __launch_bounds__(256, 3) void route_select16_kernel(
    const uint16_t* __restrict__ dq16, const void* __restrict__ g, const float* __restrict__ sg,
    const float* __restrict__ lz, int nt, int group, int g0, int ng, int nb, int nb_pad, int kx, int sink,
    int stride, int32_t* __restrict__ idx, float* __restrict__ rowmax) {
    extern __shared__ uint32_t keys16[];      // [nb]
    __shared__ TopkSmem sm;
    __shared__ float red_m[4][64];
    constexpr int S16_RING = 3, S16_SLOT = 2048 + 128;
    __shared__ __align__(16) char s16ring[4][FP8 ? S16_RING : 1][FP8 ? S16_SLOT : 16];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    const uint32_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int gi = (int)(blk % (uint32_t)ng), h = (int)(blk / (uint32_t)ng);
    const int64_t gs = (int64_t)h * ng + gi;  // state / idx row (the launch's window)
    constexpr int TR = 16 * NRB;              // rows per tile
    const int ts = TR / stride;
    bool first = true;
    for (int j = 0; j < group; ++j) {
        const int t = (g0 + gi) * group + j;
        if (t >= nt) break;                   // padded tiles repeat the last one
        const int64_t th = (int64_t)h * nt + t;
        u32x4 b[NRB][4];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const int r = 16 * rb + col;
            const int64_t p = th * TR + (int64_t)(r < ts ? r : 0) * stride;   // rows past ts repeat row 0
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) b[rb][ks] = *(const u32x4*)(dq16 + p * D + 32 * ks + 8 * grp);
        }
        float rmax[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) rmax[rb] = -INFINITY;
        // the wave's 16-leaf groups c = 16 w, 16 w + 64, ..: bf16 state rows are fetched into
        // registers while the previous group's products run (two register sets; a third, two
        // groups ahead, spills at three waves per SIMD and measured slower: 1.16 against 1.56
        // ms at cfg3); fp8 rows stream through a ring in LDS (below)
        using AT = std::conditional_t<FP8, u32x2, u32x4>;   // 8 e4m3 codes / 8 bf16 of a row chunk
        struct Grp {
            AT a[4];
            f32x4 sgv, lzv;
        };
        auto fetch = [&](Grp& gr, int c) {
            const int64_t s0 = gs * nb_pad + c;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if constexpr (FP8) gr.a[ks] = *(const u32x2*)((const uint8_t*)g + (s0 + col) * D + 32 * ks + 8 * grp);
                else gr.a[ks] = *(const u32x4*)((const uint16_t*)g + (s0 + col) * D + 32 * ks + 8 * grp);
            }
            gr.sgv = FP8 ? *(const f32x4*)(sg + s0 + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
            gr.lzv = *(const f32x4*)(lz + s0 + 4 * grp);
        };
        auto consume = [&](const Grp& gr, int c) {
            // the products of state_qk, in its order
            f32x4 acc[NRB];
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if constexpr (FP8) {
                    const u32x4 A = e4m3x8_to_h8_cvt(gr.a[ks]);
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb) acc[rb] = mfma_f16(A, b[rb][ks], acc[rb]);
                } else {
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb)
                        acc[rb] = mfma_bf16(as_bf16x8(gr.a[ks]), as_bf16x8(b[rb][ks]), acc[rb]);
                }
            }
            const f32x4 sgv = gr.sgv, lzv = gr.lzv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sc = __fmul_rn(sgv[i], 256.0f);
                float best = -INFINITY;
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) {
                    const float x = FP8 ? __fmul_rn(acc[rb][i], sc) : acc[rb][i];
                    best = fmaxf(best, x);
                    rmax[rb] = fmaxf(rmax[rb], __fadd_rn(x, lzv[i]));
                }
                best = col_max(best);
                const int l = c + 4 * grp + i;
                if (col == 0 && l < nb) {     // leaf l is always this lane's: no race across tiles
                    const uint32_t key = l < sink ? 0xffffffffu : order_key(__fadd_rn(best, lzv[i]));
                    keys16[l] = first ? key : max(keys16[l], key);
                }
            }
        };
        const int cw = 16 * w;
        if constexpr (FP8) {
            // fp8: each wave streams its groups through its own 3-slot LDS ring by direct loads,
            // two groups ahead (the wave reads only what it loaded: no barriers).  Slot: 16 rows
            // of 128 code bytes, chunk k of row r at 16-byte position k ^ sw8(r), then sg (64 B)
            // and lz (64 B); lane L of load i (rows 8 i + L / 8) gets position L % 8 of its row,
            // chunk (L % 8) ^ ((L / 16) % 4) ^ 4 i.
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)   // the row operands land before the first direct load
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) asm volatile("" : : "v"(b[rb][ks]));
            const uint32_t ring_w = lds_addr(&s16ring[w][0][0]);
            const uint32_t voff = (uint32_t)((lane >> 3) * D + 16 * ((lane & 7) ^ ((lane >> 4) & 3)));
            const int ngr = cw < nb ? (nb - cw + 63) / 64 : 0;
            auto issue = [&](int gj) {
                if (gj >= ngr) return;
                const int64_t s0 = gs * nb_pad + cw + 64 * gj;
                const uint32_t slot = ring_w + (uint32_t)(gj % S16_RING) * S16_SLOT;
                dma16s((const uint8_t*)g + s0 * D, voff, slot);
                dma16s((const uint8_t*)g + (s0 + 8) * D, voff ^ 64u, slot + 1024);
                if (lane < 8) dma16(lane < 4 ? sg + s0 + 4 * lane : lz + s0 + 4 * (lane - 4), slot + 2048);
            };
#pragma unroll
            for (int gj = 0; gj < S16_RING - 1; ++gj) issue(gj);
            for (int gj = 0; gj < ngr; ++gj) {
                if (gj + 1 < ngr) wait_vmcnt<3>();          // the next group's loads stay in flight
                else wait_vmcnt<0>();
                const char* slot = &s16ring[w][gj % S16_RING][0];
                Grp x;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int kc = 2 * ks + (grp >> 1);
                    x.a[ks] = *(const u32x2*)(slot + col * D + 16 * (kc ^ sw8(col)) + 8 * (grp & 1));
                }
                x.sgv = *(const f32x4*)(slot + 2048 + 16 * grp);
                x.lzv = *(const f32x4*)(slot + 2048 + 64 + 16 * grp);
                issue(gj + S16_RING - 1);                    // into the slot read last iteration
                consume(x, cw + 64 * gj);
            }
        } else {
            Grp x0, x1;
            if (cw < nb) fetch(x0, cw);
            for (int c = cw; c < nb; c += 128) {
                if (c + 64 < nb) fetch(x1, c + 64);
                consume(x0, c);
                if (c + 64 >= nb) break;
                if (c + 128 < nb) fetch(x0, c + 128);
                consume(x1, c + 64);
            }
        }
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const float mx = grp_max(rmax[rb]);
            if (grp == 0) red_m[w][16 * rb + col] = mx;
        }
        __syncthreads();
        if (w == 0) {
            const int r = lane;
            float m = r < ts ? fmaxf(fmaxf(red_m[0][r], red_m[1][r]), fmaxf(red_m[2][r], red_m[3][r])) : -INFINITY;
            if (stride != 1) m = wave_max(m); // sampled rows: one reference for the whole tile
            if (r < TR) rowmax[th * TR + r] = m;
        }
        __syncthreads();                      // red_m is free for the next tile of the group
        first = false;
    }
    const int kxe = min(kx, nb);
    if (kxe > 0) topk_row([&](int l) { return keys16[l]; }, nb, kxe, sm, idx + gs * kxe, nullptr, nullptr);
}

// One ring slot of route16_kernel: QK rows and PV rows, 32 rows of 128 16-bit values each, then
// the far block's 32-float scale vectors (lz; for fp8 also sg and sv, as stored).  PV row r keeps
// its 16-byte chunk c at c ^ swz(r) (the transposing reads); QK row r at c ^ swq(r), so that the
// QK operand reads (16 rows at one chunk) hit 16 different chunks and every 8 consecutive rows 8
// different chunks modulo 8: no bank conflicts in 8- or 16-lane phases.  An fp8 far block fills
// the first 4 KiB of each region: 32 rows of 128 codes, chunk c of row r at c ^ sw8(r) (its QK
// reads touch rows 16 h + 0..15 per 32 lanes, its PV reads rows 4 g + 0..3, 16 + 4 g + 0..3).
constexpr int R16_ROWS = 32 * 256;
constexpr int R16_SLOT = 2 * R16_ROWS + 3 * 32 * 4;
__device__ __forceinline__ int swq(int r) { return r & 15; }

// p = 2^u for the log2-domain shifted scores u[rb][0..7] of the RB row blocks (keys 16(e/4) + 4grp
// + e%4), l += p, O^T += V^T P^T with P = fp16(p * pscale) per key (the fp8 far field).
template <int RB, typename VOp>
__device__ __forceinline__ void rows_update_f16(RowsN<RB>& st, const float (&u)[RB][8], const float (&pscale)[8],
                                                VOp vop) {
    u32x4 P[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(u[rb][e]);
        st.l[rb] = __fadd_rn(st.l[rb], __fadd_rn(__fadd_rn(__fadd_rn(p[0], p[1]), __fadd_rn(p[2], p[3])),
                                                 __fadd_rn(__fadd_rn(p[4], p[5]), __fadd_rn(p[6], p[7]))));
        uint32_t ph[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ph[j] = pack2h(__fmul_rn(p[2 * j], pscale[2 * j]), __fmul_rn(p[2 * j + 1], pscale[2 * j + 1]));
        P[rb] = u32x4{ph[0], ph[1], ph[2], ph[3]};
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        if (db == 4) __builtin_amdgcn_sched_barrier(0);   // at most half the V^T operands in registers
        const u32x4 A = vop(db);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) st.o[rb][db] = mfma_f16(A, P[rb], st.o[rb][db]);
    }
}

// rows_update with the V^T operand of dims block db read by vop(db) as it is consumed.
template <int RB, typename VOp>
__device__ __forceinline__ void rows_update_bf16(RowsN<RB>& st, const float (&sc)[RB][8], VOp vop) {
    bf16x8 P[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(sc[rb][e]);
        st.l[rb] = __fadd_rn(st.l[rb], __fadd_rn(__fadd_rn(__fadd_rn(p[0], p[1]), __fadd_rn(p[2], p[3])),
                                                 __fadd_rn(__fadd_rn(p[4], p[5]), __fadd_rn(p[6], p[7]))));
        P[rb] = to_bf16x8(p);
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
        if (db == 4) __builtin_amdgcn_sched_barrier(0);   // at most half the V^T operands in registers
        const bf16x8 A = as_bf16x8(vop(db));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) st.o[rb][db] = mfma_bf16(A, P[rb], st.o[rb][db]);
    }
}

// The largest score (log2 units) of each of this wave's rows (prowb + 16 rb + col, prowb
// wave-uniform) over every key it
// attends in route16_kernel: the far leaves not excluded, then the near tokens, 16 keys at a time
// with both MFMA operands loaded straight from global memory; every lane of a row's column ends
// with it.  It runs only when a tile's reference missed; lane-dependent addresses come from a
// lane index redefined through an empty asm (route_exact_max).
template <int LEAF, bool FP8, int RB>
__device__ __forceinline__ RowMax<RB> route16_exact_max(const uint16_t* dq16, const uint16_t* q16, const void* g,
                                                     const float* sg, const float* lz, const uint32_t* exbits,
                                                     int64_t srow0, int nb, const uint16_t* k, const uint32_t* sidx,
                                                     int64_t kh, int e_n, int64_t prowb, float qs) {
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const int col = lane & 15, grp = lane >> 4;
    const int64_t prow0 = prowb + col;
    RowMax<RB> mx;
    u32x4 bx[RB][4];
    auto load_rows = [&](const uint16_t* x) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) bx[rb][ks] = *(const u32x4*)(x + (prow0 + 16 * rb) * D + 32 * ks + 8 * grp);
    };
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) mx.m[rb] = -INFINITY;
    load_rows(dq16);
    for (int c = 0; c < nb; c += 16) {            // rows < nb_pad; leaves >= nb are excluded
        const int64_t r = srow0 + c;
        f32x4 acc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int64_t off = (r + col) * D + 32 * ks + 8 * grp;
            const u32x4 A = FP8 ? e4m3x8_to_h8_cvt(*(const u32x2*)((const uint8_t*)g + off))
                                : *(const u32x4*)((const uint16_t*)g + off);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if constexpr (FP8) acc[rb] = mfma_f16(A, bx[rb][ks], acc[rb]);
                else acc[rb] = mfma_bf16(as_bf16x8(A), as_bf16x8(bx[rb][ks]), acc[rb]);
            }
        }
        const f32x4 lzv = *(const f32x4*)(lz + r + 4 * grp);
        const f32x4 sgv = FP8 ? *(const f32x4*)(sg + r + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
        const uint32_t exw = exbits[c >> 5] >> ((c & 31) + 4 * grp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float lzi = (exw >> i) & 1u ? -INFINITY : lzv[i];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                // fp8: the widened codes are value * 2^-8, the row scale enters * 256 (exactly)
                const float dot = FP8 ? __fmul_rn(acc[rb][i], __fmul_rn(sgv[i], 256.0f)) : acc[rb][i];
                mx.m[rb] = fmaxf(mx.m[rb], __fmul_rn(__fadd_rn(dot, lzi), LOG2E));
            }
        }
    }
    load_rows(q16);
    for (int j = 0; j < e_n; j += 16) {           // 16-token runs of the near leaves
        const int64_t tok = kh + (int64_t)__builtin_amdgcn_readfirstlane(sidx[j / LEAF]) * LEAF + (j % LEAF);
        f32x4 acc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const u32x4 A = *(const u32x4*)(k + (tok + col) * D + 32 * ks + 8 * grp);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma_bf16(as_bf16x8(A), as_bf16x8(bx[rb][ks]), acc[rb]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) mx.m[rb] = fmaxf(mx.m[rb], __fmul_rn(acc[rb][i], qs));
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) mx.m[rb] = grp_max(mx.m[rb]);
    return mx;
}

template <int LEAF, bool FP8, int NW, int RB>
__global__ __launch_bounds__(64 * NW, 2) void route16_kernel(
    const uint16_t* __restrict__ q16, const uint16_t* __restrict__ dq16, const void* __restrict__ g,
    const float* __restrict__ sg, const float* __restrict__ lz, const void* __restrict__ vb,
    const float* __restrict__ sv, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ idx, const float* __restrict__ rowmax, int64_t nq, int nt, int group, int g0, int ng,
    const int32_t* __restrict__ perm, int64_t nk, int nb, int nb_pad, int kxe, float scale,
    float* __restrict__ out, float* __restrict__ logz) {
    static_assert(NW == 2, "two waves per tile: wave w stages rows 16 w .. 16 w + 15 of every block");
    constexpr int NT = 64 * NW, TR = 16 * RB * NW;   // threads, rows per tile (16 RB rows per wave)
    __shared__ __align__(16) char ring[2][R16_SLOT];
    // sized by the launch: exclusion bits [nb / 32 + 1], then the tile's near leaves [kxe]
    extern __shared__ __align__(16) uint32_t r16_dyn[];
    uint32_t* exbits = r16_dyn;
    uint32_t* sidx = r16_dyn + (nb / 32 + 1);
    __shared__ float red_l[TR];
    __shared__ int redo;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
    // 1-D grid over (tile, head), tile fastest (route_kernel's XCD-contiguous order); the tiles of
    // groups [g0, g0 + ng), state and idx rows the launch's own
    const int tb = g0 * group, ntw = min(nt, (g0 + ng) * group) - tb;
    const uint32_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int t = tb + (int)(blk % (uint32_t)ntw), h = (int)(blk / (uint32_t)ntw);
    const int64_t th = (int64_t)h * nt + t;
    const int64_t gs = (int64_t)h * ng + (t / group - g0);
    const int64_t kh = (int64_t)h * nk;
    const int64_t prow0 = th * TR + 16 * RB * wv + col;     // this lane's packed query row of block 0
    for (int i = threadIdx.x; i <= nb / 32; i += NT) {     // leaves >= nb excluded
        const int past = nb - 32 * i;
        exbits[i] = past >= 32 ? 0u : (past <= 0 ? ~0u : ~0u << past);
    }
    for (int j = threadIdx.x; j < kxe; j += NT) sidx[j] = (uint32_t)idx[gs * kxe + j];
    float mref[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float m = rowmax[prow0 + 16 * rb];
        mref[rb] = m == -INFINITY ? 0.0f : __fmul_rn(m, LOG2E);
    }
    // B operands of the rows: q - mu through the far blocks, then q through the near blocks (one
    // register set, reloaded at the switch)
    u32x4 bx[RB][4];
    auto load_rows = [&](const uint16_t* x) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) bx[rb][ks] = *(const u32x4*)(x + (prow0 + 16 * rb) * D + 32 * ks + 8 * grp);
    };
    __syncthreads();
    for (int j = threadIdx.x; j < kxe; j += NT) atomicOr(&exbits[sidx[j] >> 5], 1u << (sidx[j] & 31));
    __syncthreads();
    const int nf = (nb + 31) / 32;                          // far blocks of 32 leaves (rows < nb_pad)
    const int e_n = kxe * LEAF;
    const int nn = (e_n + 31) / 32;                         // near blocks: two 16-token runs each
    const int nblk = nf + nn;
    const float qs = __fmul_rn(scale, LOG2E);
    // Direct global -> LDS loads of 256-byte rows: wave w stages rows 16 w .. 16 w + 15 of a block's
    // QK and PV regions, four rows per load; lane L of load i gets row 4 i + L / 16 at position
    // L % 16, i.e. the row's 16-byte chunk (L % 16) ^ swq (QK) or ^ swz (PV) of that row.
    // With g = L / 16 and r = 4 i + g (bits of i above those of g): swq(r) = 4 i ^ g and
    // swz(r) = (g << 1) ^ f(i), f = 0, 9, 8, 1, so load i's offsets are load 0's XOR a constant.
    // The per-block lambdas derive their lane offsets from ln, which every pass redefines through
    // an empty asm: otherwise those offsets are hoisted out of the pass loop and all of them stay
    // live (and spill) through both key loops.
    int ln = lane;
    auto dma_rows16 = [&](const uint16_t* xq, const uint16_t* xp, uint32_t slot_lds) {
        const uint32_t voq0 = (uint32_t)((ln >> 4) * 256 + 16 * ((ln & 15) ^ swq(ln >> 4)));
        const uint32_t vop0 = (uint32_t)((ln >> 4) * 256 + 16 * ((ln & 15) ^ swz(ln >> 4)));
        const uint64_t bq_ = sbase(xq), bp_ = sbase(xp);
        const uint32_t lq = slot_lds + (uint32_t)wv * 4096, lp = slot_lds + R16_ROWS + (uint32_t)wv * 4096;
        dma_x4<false>(bq_, voq0, bq_, voq0 ^ 64u, bq_, voq0 ^ 128u, bq_, voq0 ^ 192u, lq);
        dma_x4<false>(bp_, vop0, bp_, vop0 ^ 144u, bp_, vop0 ^ 128u, bp_, vop0 ^ 16u, lp);
    };
    // fp8 far blocks: the code rows (128 bytes) as they are, chunk c of row r at 16-byte
    // position c ^ sw8(r) of the QK and PV regions (rows 128 bytes apart), widened to fp16 as
    // they are read.  Lane L of load i (rows 16 w + 8 i + L / 8) gets position L % 8 of its row,
    // chunk (L % 8) ^ sw8(row) = (L % 8) ^ ((L / 16) % 4) ^ 4 (i ^ w).
    auto dma_rows8 = [&](const uint8_t* xq, const uint8_t* xp, uint32_t slot_lds) {
        const uint32_t vo = (uint32_t)((ln >> 3) * D + 16 * ((ln & 7) ^ ((ln >> 4) & 3) ^ (4 * wv)));
        const uint32_t lq = slot_lds + (uint32_t)wv * 2048, lp = slot_lds + R16_ROWS + (uint32_t)wv * 2048;
        dma16s(xq, vo, lq);
        dma16s(xq + 8 * D, vo ^ 64u, lq + 1024);
        dma16s(xp, vo, lp);
        dma16s(xp + 8 * D, vo ^ 64u, lp + 1024);
    };
    auto run_pos = [&](int j) { return j < e_n ? j : 0; };  // past the list: its start again (masked)
    // near block bi (tokens of the near list from 32 (bi - nf)): wave w loads the 16-token run
    // 32 (bi - nf) + 16 w (past the list: the list's start again, masked)
    auto fetch_near = [&](int bi, uint32_t sl_lds) {
        const int e0 = 32 * (bi - nf) + 16 * wv, j = run_pos(e0);
        const int64_t ra = kh + (int64_t)__builtin_amdgcn_readfirstlane(sidx[j / LEAF]) * LEAF + (j % LEAF);
        dma_rows16(k + ra * D, v + ra * D, sl_lds);
    };
    // Block bi into ring slot `slot` by direct loads (landed once this wave's vmcnt drains): a
    // far block (its rows 16 w .. of g and vb from wave w; lz, and for fp8 sg and sv, from wave 0)
    // or a near block.
    auto fetch = [&](int bi, int slot) {
        char* sl = &ring[slot][0];
        const uint32_t sl_lds = lds_addr(sl);
        if (bi < nf) {                                      // 32 consecutive state rows of the group
            const int64_t r0 = gs * nb_pad + 32 * bi;
            const int64_t rw = r0 + 16 * wv;
            if constexpr (FP8) {
                dma_rows8((const uint8_t*)g + rw * D, (const uint8_t*)vb + rw * D, sl_lds);
                if (wv == 0 && lane < 8) {
                    dma16s<false>(lz + r0, (uint32_t)(16 * lane), sl_lds + 2 * R16_ROWS);
                    dma16s<false>(sg + r0, (uint32_t)(16 * lane), sl_lds + 2 * R16_ROWS + 128);
                    dma16s<false>(sv + r0, (uint32_t)(16 * lane), sl_lds + 2 * R16_ROWS + 256);
                }
            } else {
                dma_rows16((const uint16_t*)g + rw * D, (const uint16_t*)vb + rw * D, sl_lds);
                if (wv == 0 && lane < 8) dma16s<false>(lz + r0, (uint32_t)(16 * lane), sl_lds + 2 * R16_ROWS);
            }
        } else {
            fetch_near(bi, sl_lds);
        }
    };
    RowsN<RB> st;
    // one 32-key block of the far field: score = (dq . g) (* 256 sg) + lz; each LDS operand read
    // feeds the RB row blocks
    auto far_block = [&](const char* slot, int bi) {
        const int col = ln & 15, grp = ln >> 4, lane = ln;
        float u[RB][8], pscale[8];
        const float* scl = (const float*)(slot + 2 * R16_ROWS);
        const uint32_t exw = exbits[bi] >> (4 * grp);      // excluded leaves: lz -> -inf below
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (hh == 1) __builtin_amdgcn_sched_barrier(0);   // one key half's QK operands at a time
            const int r = 16 * hh + col;
            f32x4 acc[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                u32x4 A;
                if constexpr (FP8) {   // eight codes of row r, dims 32 ks + 8 grp ..: chunk 2 ks + grp / 2
                    const int kc = 2 * ks + (grp >> 1);
                    A = e4m3x8_to_h8_cvt(*(const u32x2*)(slot + r * D + 16 * (kc ^ sw8(r)) + 8 * (grp & 1)));
                } else {
                    A = *(const u32x4*)(slot + r * 256 + 16 * ((4 * ks + grp) ^ swq(r)));
                }
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    if constexpr (FP8) acc[rb] = mfma_f16(A, bx[rb][ks], acc[rb]);
                    else acc[rb] = mfma_bf16(as_bf16x8(A), as_bf16x8(bx[rb][ks]), acc[rb]);
                }
            }
            const f32x4 lzv = *(const f32x4*)(scl + 16 * hh + 4 * grp);
            const f32x4 sgv = FP8 ? *(const f32x4*)(scl + 32 + 16 * hh + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
            const f32x4 svv = FP8 ? *(const f32x4*)(scl + 64 + 16 * hh + 4 * grp) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // excluded key: lz -> -inf, one bit select on the sign-extended bit
                const uint32_t ex = (uint32_t)__builtin_amdgcn_sbfe((int)exw, 16 * hh + i, 1);
                uint32_t lzb;
                asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(lzb) : "v"(ex), "v"(0xff800000u), "v"(__float_as_uint(lzv[i])));
                const float lzi = __uint_as_float(lzb);
                // fp8: the widened codes are value * 2^-8, so the row scales enter * 256 (exactly)
                const float sgi = FP8 ? __fmul_rn(sgv[i], 256.0f) : 1.0f;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    const float dot = FP8 ? __fmul_rn(acc[rb][i], sgi) : acc[rb][i];
                    u[rb][4 * hh + i] = __fmaf_rn(__fadd_rn(dot, lzi), LOG2E, -st.m[rb]);
                }
                pscale[4 * hh + i] = FP8 ? __fmul_rn(svv[i], 256.0f) : 1.0f;
            }
        }
        if constexpr (FP8) {
            // V^T of dims 16 db + L % 16 at the keys of P's k-items in lane group grp (4 grp + 0..3,
            // then 16 + 4 grp + 0..3: the QK accumulator layout): lanes 2 j, 2 j + 1 of the group
            // address the two halves of chunk db of the j-th of those key rows; the transposing byte
            // read hands lane L that dim of the eight rows, widened to fp16
            auto vop8 = [&](int db) {
                const int j = col >> 1, rw8 = 4 * grp + (j & 3) + 16 * (j >> 2);
                return e4m3x8_to_h8_cvt(lds_read_tr8(slot + R16_ROWS + rw8 * D + 16 * (db ^ sw8(rw8)) + 8 * (col & 1)));
            };
            rows_update_f16<RB>(st, u, pscale, vop8);
        } else {
            auto vop_ = [&](int db) {
                const u32x2 lo = tr_operand(slot + R16_ROWS, 0, db, lane), hi = tr_operand(slot + R16_ROWS, 16, db, lane);
                return u32x4{lo.x, lo.y, hi.x, hi.y};
            };
            rows_update_bf16<RB>(st, u, vop_);
        }
    };
    // one 32-token block of the near field: score = (q . k) * scale; the second run of 16 is past
    // the list (masked) only in the last block when the list holds an odd number of 16-token runs
    auto near_block = [&](const char* slot, int bi) {
        const int col = ln & 15, grp = ln >> 4, lane = ln;
        const bool run2 = 32 * (bi - nf) + 16 < e_n;
        float u[RB][8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (hh == 1) __builtin_amdgcn_sched_barrier(0);   // one key half's QK operands at a time
            const int r = 16 * hh + col;
            f32x4 acc[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const u32x4 A = *(const u32x4*)(slot + r * 256 + 16 * ((4 * ks + grp) ^ swq(r)));
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma_bf16(as_bf16x8(A), as_bf16x8(bx[rb][ks]), acc[rb]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    u[rb][4 * hh + i] = (hh == 0 || run2) ? __fmaf_rn(acc[rb][i], qs, -st.m[rb]) : -INFINITY;
        }
        auto vop_ = [&](int db) {
            const u32x2 lo = tr_operand(slot + R16_ROWS, 0, db, lane), hi = tr_operand(slot + R16_ROWS, 16, db, lane);
            return u32x4{lo.x, lo.y, hi.x, hi.y};
        };
        rows_update_bf16<RB>(st, u, vop_);
    };
    // block bi from slot S while block bi + 1 is fetched into the other slot; the step ends with
    // both waves' loads landed
    auto far_step = [&](auto par, int bi) {
        constexpr int S = decltype(par)::value;
        if (bi + 1 < nblk) fetch(bi + 1, S ^ 1);
        far_block(&ring[S][0], bi);
        wait_vmcnt<0>();
        __syncthreads();
    };
    auto near_step = [&](auto par, int bi) {
        constexpr int S = decltype(par)::value;
        if (bi + 1 < nblk) fetch_near(bi + 1, lds_addr(&ring[S ^ 1][0]));
        near_block(&ring[S][0], bi);
        wait_vmcnt<0>();
        __syncthreads();
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    for (int pass = 0; pass < MAX_PASSES; ++pass) {
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            st.m[rb] = mref[rb];
            st.l[rb] = 0.0f;
#pragma unroll
            for (int db = 0; db < 8; ++db) st.o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        load_rows(dq16);
        // the row operands are in registers before the first direct load (the compiler's own wait
        // for them would otherwise also drain it)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) asm volatile("" : : "v"(bx[rb][ks]));
        fetch(0, 0);
        wait_vmcnt<0>();
        __syncthreads();
        // far blocks 0 .. nf - 1 in slots 0, 1, 0, ..; the near blocks continue the alternation
        for (int bi = 0; bi < nf; bi += 2) {
            far_step(P0(), bi);
            if (bi + 1 < nf) far_step(P1(), bi + 1);
        }
        load_rows(q16);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) asm volatile("" : : "v"(bx[rb][ks]));
        if (nf & 1) {
            for (int bi = nf; bi < nblk; bi += 2) {
                near_step(P1(), bi);
                if (bi + 1 < nblk) near_step(P0(), bi + 1);
            }
        } else {
            for (int bi = nf; bi < nblk; bi += 2) {
                near_step(P0(), bi);
                if (bi + 1 < nblk) near_step(P1(), bi + 1);
            }
        }
        // row totals: outside [2^-60, 2^64] the reference missed the row's maximum by more than 60
        // octaves (2^-8 with the fp8 store: its far-field P is fp16, whose subnormals would hold
        // the far leaves of a row whose total is that small with too few bits): the tile is redone
        // once at every row's exact largest score, where each row total lies in [1, keys]
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float lt = grp_sum(st.l[rb]);
            if (grp == 0) red_l[16 * RB * wv + 16 * rb + col] = lt;
        }
        if (threadIdx.x == 0) redo = 0;
        __syncthreads();
        bool bad = false;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float tot = red_l[16 * RB * wv + 16 * rb + col];
            if (!(tot >= (FP8 ? 0x1p-8f : 0x1p-60f) && tot <= 0x1p64f)) bad = true;
        }
        if (bad) redo = 1;
        __syncthreads();
        if (__builtin_expect(redo == 0 || pass + 1 == MAX_PASSES, 1)) break;
        const RowMax<RB> mx = route16_exact_max<LEAF, FP8, RB>(dq16, q16, g, sg, lz, exbits, gs * nb_pad, nb, k, sidx,
                                                              kh, e_n, th * TR + 16 * RB * wv, qs);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
            if (mx.m[rb] > -INFINITY) mref[rb] = mx.m[rb];
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * RB * wv + 16 * rb + col;
        const float den = red_l[r];
        const float inv = 1.0f / (den < 1e-30f ? 1e-30f : den);
        const int64_t qi = (int64_t)t * TR + r;
        if (qi < nq) {
            const int64_t orow = (int64_t)h * nq + perm_row(perm, h, nq, qi);
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const f32x4 o = st.o[rb][db];
                *(f32x4*)(out + orow * D + 16 * db + 4 * grp) =
                    f32x4{__fmul_rn(o[0], inv), __fmul_rn(o[1], inv), __fmul_rn(o[2], inv), __fmul_rn(o[3], inv)};
            }
            if (grp == 0) logz[orow] = __fadd_rn(__fmul_rn(st.m[rb], LN2), __logf(den));   // m in log2 units
        }
    }
}

// ---------------------------------------------------------------------------------------------
// tail: keys past the last full leaf, attended exactly by every query, merged into a finished
// (out, logz).  The reference folds up to 16 such keys into the last split of its tile kernel
// with q, k, v and p rounded to bf16 (h3/htrc_flat_triton.py:187-207) and takes a host-side fp32
// partial for more (:381-388); both end as one softmax over far, near and tail, which is what
// the log-sum-exp merge here computes.  Four lanes per query row (32 dims each).
// ---------------------------------------------------------------------------------------------
// MODE 0: the dot="bf16" paths (up to 16 keys in bf16, more in fp32); 1: fp32 operands; 2: TF32
// operands (the fp32-dot path, h3/htrc_flat_triton.py:198-207 with DOT = 0).
template <bool IN_BF16, int MODE = 0>
__global__ __launch_bounds__(256) void tail_kernel(const void* __restrict__ q, const float* __restrict__ tk,
                                                   const float* __restrict__ tv, int64_t nq, int ntail,
                                                   float scale, float* __restrict__ out, float* __restrict__ logz) {
    const int t = blockIdx.x, h = blockIdx.y, r = threadIdx.x >> 2, qd = threadIdx.x & 3;
    const int64_t qi = (int64_t)t * TILE + r;
    if (qi >= nq) return;                         // whole 4-lane groups leave together
    const bool bfr = MODE == 0 && ntail <= 16;    // the in-kernel path of the reference works in bf16
    auto op = [&](float x) { return bfr ? bf16_round(x) : (MODE == 2 ? tf32_rna(x) : x); };
    const int64_t row = (int64_t)h * nq + qi;
    float qv[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const float x = IN_BF16 ? bf2f(((const uint16_t*)q)[row * D + 32 * qd + e]) : ((const float*)q)[row * D + 32 * qd + e];
        qv[e] = op(x);
    }
    auto score = [&](int j) {                     // (q . k_j) * scale, the row's four lanes together
        const float* kj = tk + ((int64_t)h * ntail + j) * D + 32 * qd;
        float sdot = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) sdot = fmaf(qv[e], op(kj[e]), sdot);
        sdot = __fadd_rn(sdot, __shfl_xor(sdot, 1, 4));
        sdot = __fadd_rn(sdot, __shfl_xor(sdot, 2, 4));
        return __fmul_rn(sdot, scale);
    };
    // two passes: p = exp(s - max over the tail), so its bf16 rounding does not depend on key order
    float m = -INFINITY;
    for (int j = 0; j < ntail; ++j) m = fmaxf(m, score(j));
    float l = 0.0f, acc[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = 0.0f;
    for (int j = 0; j < ntail; ++j) {
        const float* vj = tv + ((int64_t)h * ntail + j) * D + 32 * qd;
        const float p = expf(__fsub_rn(score(j), m));
        l = __fadd_rn(l, p);
        const float pv = op(p);
#pragma unroll
        for (int e = 0; e < 32; ++e) acc[e] = fmaf(pv, op(vj[e]), acc[e]);
    }
    const float lse = __fadd_rn(m, logf(l));
    const float lz0 = logz[row];
    const float mx = fmaxf(lz0, lse);
    const float nz = __fadd_rn(mx, logf(__fadd_rn(expf(__fsub_rn(lz0, mx)), expf(__fsub_rn(lse, mx)))));
    const float w0 = expf(__fsub_rn(lz0, nz)), w1 = __fdiv_rn(expf(__fsub_rn(lse, nz)), l);
    float* o = out + row * D + 32 * qd;
#pragma unroll
    for (int e = 0; e < 32; e += 4) {
        const f32x4 x = *(const f32x4*)(o + e);
        *(f32x4*)(o + e) = f32x4{fmaf(acc[e], w1, __fmul_rn(x[0], w0)), fmaf(acc[e + 1], w1, __fmul_rn(x[1], w0)),
                                 fmaf(acc[e + 2], w1, __fmul_rn(x[2], w0)), fmaf(acc[e + 3], w1, __fmul_rn(x[3], w0))};
    }
    if (qd == 0) logz[row] = nz;
}

// ---------------------------------------------------------------------------------------------
// selftest_mfma: one wave computes C = A B with the operand conventions used above
// (A row m = lane%16 with k-set lane/16, B column n = lane%16 with the same k-set,
// C[4*(lane/16) + i][lane%16] in item i).
// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// k-means query order (h3/htrc_flat.py:47-61): Lloyd's k-means on an even sample of the
// queries, every query assigned to its nearest centre, and the rows ordered by centre (stable).
//   sample i: row round(linspace(0, n - 1, m)[i]), m = min(sample, n), in torch's float32
//   device linspace (step = (n - 1) / (m - 1); i < m / 2: i step, else the fused
//   (n - 1) - (m - 1 - i) step), rounded to nearest even; initial centre j: sample
//   round(linspace(0, m - 1, C)[j]).
//   distance: sequential fp32 sum over the dims of (x - c)^2, ties to the lower centre (the
//   reference ranks sqrt of the matrix-product form; both give the same order except where
//   two centres tie to rounding).
//   update: per centre, the sequential fp32 sum of its samples in sample order divided by their
//   count; a centre without samples keeps its position.
// ---------------------------------------------------------------------------------------------
constexpr int KM_MAX_C = 64;           // clusters
constexpr int KM_MAX_SAMPLE = 16384;   // sample rows

__device__ __forceinline__ int64_t linspace_round(int64_t hi, int64_t steps, int64_t i) {
    if (steps <= 1) return 0;
    const float step = __fdiv_rn((float)hi, (float)(steps - 1));
    // lower half step * i; upper half hi - step * (steps - 1 - i) in one fused multiply-add, as
    // torch's device kernel computes it (checked against torch.linspace on this GPU)
    const float v = i < steps / 2 ? __fmul_rn(step, (float)i) : __fmaf_rn(-step, (float)(steps - 1 - i), (float)hi);
    const int64_t r = (int64_t)rintf(v);
    return r < 0 ? 0 : (r > hi ? hi : r);      // (float)hi may round above hi for hi >= 2^24
}

template <bool IN_BF16>
__device__ __forceinline__ float qval(const void* q, int64_t idx) {
    return IN_BF16 ? bf2f(((const uint16_t*)q)[idx]) : ((const float*)q)[idx];
}

template <bool IN_BF16>
__global__ __launch_bounds__(128) void km_init_kernel(const void* __restrict__ q, int64_t nq, int m, int C,
                                                      float* __restrict__ cen) {
    const int j = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
    const int64_t row = linspace_round(nq - 1, m, linspace_round(m - 1, C, j));
    cen[((int64_t)h * C + j) * D + i] = qval<IN_BF16>(q, ((int64_t)h * nq + row) * D + i);
}

// Nearest centre of 256 rows (of the sample when sm > 0, else of the queries): one row per
// lane, its 128 values in registers.  The centres are wave-uniform: read straight from memory
// (scalar loads into operands, no per-lane copies), four centres per step as independent sums
// (then pairs, then one), compared in increasing order so that ties keep the lower centre.
template <bool IN_BF16>
__global__ __launch_bounds__(256) void km_assign_kernel(const void* __restrict__ q, int64_t nq, int64_t nrows, int sm,
                                                        int C, const float* __restrict__ cen,
                                                        int32_t* __restrict__ assign) {
    const int h = blockIdx.y, tid = threadIdx.x;
    const float* __restrict__ ch = cen + (int64_t)h * C * D;
    const int64_t ri = (int64_t)blockIdx.x * 256 + tid;
    const int64_t rc = ri < nrows ? ri : nrows - 1;
    const int64_t row = sm > 0 ? linspace_round(nq - 1, sm, rc) : rc;
    const int64_t base = ((int64_t)h * nq + row) * D;
    float x[D];
    if constexpr (IN_BF16) {
#pragma unroll
        for (int c8 = 0; c8 < D / 8; ++c8) {
            const u32x4 u = *(const u32x4*)((const uint16_t*)q + base + 8 * c8);
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[8 * c8 + 2 * e] = __uint_as_float(w4[e] << 16);
                x[8 * c8 + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
        for (int c4 = 0; c4 < D / 4; ++c4) {
            const f32x4 v = *(const f32x4*)((const float*)q + base + 4 * c4);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * c4 + e] = v[e];
        }
    }
    float best = INFINITY;
    int bj = C;
    auto consider = [&](float acc, int j) {
        if (acc < best) {
            best = acc;
            bj = j;
        }
    };
    int j = 0;
    for (; j + 3 < C; j += 4) {
        const float* c0 = ch + (int64_t)j * D;
        float a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float e = __fsub_rn(x[d], c0[u * D + d]);
                a[u] = __fadd_rn(a[u], __fmul_rn(e, e));
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) consider(a[u], j + u);
    }
    for (; j + 1 < C; j += 2) {
        const float* c0 = ch + (int64_t)j * D;
        const float* c1 = c0 + D;
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float e0 = __fsub_rn(x[d], c0[d]), e1 = __fsub_rn(x[d], c1[d]);
            a0 = __fadd_rn(a0, __fmul_rn(e0, e0));
            a1 = __fadd_rn(a1, __fmul_rn(e1, e1));
        }
        consider(a0, j);
        consider(a1, j + 1);
    }
    if (j < C) {                        // an odd last centre
        const float* c0 = ch + (int64_t)j * D;
        float a0 = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float e0 = __fsub_rn(x[d], c0[d]);
            a0 = __fadd_rn(a0, __fmul_rn(e0, e0));
        }
        consider(a0, j);
    }
    if (bj >= C) bj = 0;                // no finite distance (non-finite rows): centre 0
    if (ri < nrows) assign[(int64_t)h * nq + ri] = bj;
}

// New centre j: the samples assigned to j (listed in sample order by a ballot compaction, as
// their rows of q) summed in that order and divided by their count.  The assignments are read
// four 128-sample chunks ahead and compacted four chunks per barrier pair, and the rows are
// gathered 32 at a time, so that neither walk waits on one load per step.
template <bool IN_BF16>
__global__ __launch_bounds__(128) void km_update_kernel(const void* __restrict__ q, int64_t nq, int m, int C,
                                                        const int32_t* __restrict__ assign,
                                                        float* __restrict__ cen) {
    constexpr int PF = 4;
    __shared__ int32_t list[KM_MAX_SAMPLE];
    __shared__ int wcnt[2 * PF];                  // [wave][chunk] hit counts
    const int j = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int32_t* a = assign + (int64_t)h * nq;
    int pre[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const int i = 128 * p + tid;
        pre[p] = i < m ? a[i] : -1;
    }
    int cnt = 0;
    for (int i0 = 0; i0 < m; i0 += 128 * PF) {
        int cur[PF];
        uint64_t bal[PF];
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            cur[p] = pre[p];
            const int i = i0 + 128 * (PF + p) + tid;
            pre[p] = i < m ? a[i] : -1;
            bal[p] = __ballot(cur[p] == j);       // -1 past the sample
            if (lane == 0) wcnt[PF * w + p] = __popcll(bal[p]);
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < PF; ++p) {            // chunk p: wave 0's hits, then wave 1's
            if (cur[p] == j)
                list[cnt + (w ? wcnt[p] : 0) + __popcll(bal[p] & ((1ull << lane) - 1ull))] =
                    (int32_t)linspace_round(nq - 1, m, i0 + 128 * p + tid);
            cnt += wcnt[p] + wcnt[PF + p];
        }
        __syncthreads();
    }
    // dim tid of B rows per step: the raw words first (every load unconditional, indices past
    // the list repeating its first row), then the values summed in list order.
    const int64_t hb = (int64_t)h * nq * D + tid;
    float acc = 0.0f;
    constexpr int B = 32;
    for (int k0 = 0; k0 < cnt; k0 += B) {
        uint32_t raw[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int64_t e = hb + (int64_t)list[k0 + u < cnt ? k0 + u : k0] * D;
            raw[u] = IN_BF16 ? (uint32_t)((const uint16_t*)q)[e] : ((const uint32_t*)q)[e];
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const float x = IN_BF16 ? __uint_as_float(raw[u] << 16) : __uint_as_float(raw[u]);
            if (k0 + u < cnt) acc = __fadd_rn(acc, x);
        }
    }
    if (cnt > 0) cen[((int64_t)h * C + j) * D + tid] = __fdiv_rn(acc, (float)cnt);
}

// perm = the rows ordered by centre, the rows of one centre in row order: a stable counting sort
// over at most KM_SORT_RANGES row ranges of whole 1024-row chunks per head, one workgroup per
// range.  km_count_kernel writes every range's count of each centre; km_place_kernel starts
// each centre at the rows of the centres before it plus that centre's rows in earlier ranges,
// then places its range chunk by chunk with ballot ranks (one ballot per distinct centre of a
// wave, the next chunk's centres read ahead).
constexpr int KM_SORT_RANGES = 128;

// rows per range: whole 1024-row chunks, at most KM_SORT_RANGES ranges
inline int64_t km_sort_span(int64_t nq) {
    const int64_t chunks = (nq + 1023) / 1024;
    return 1024 * ((chunks + KM_SORT_RANGES - 1) / KM_SORT_RANGES);
}

__device__ __forceinline__ int km_centre(const int32_t* a, int64_t p, int C) {
    const int c = a[p];
    return c >= 0 && c < C ? c : 0;
}

// counts[h][range][c]: the rows of range `range` of head h assigned to centre c
__global__ __launch_bounds__(1024) void km_count_kernel(const int32_t* __restrict__ assign, int64_t nq, int C,
                                                        int64_t span, uint32_t* __restrict__ counts) {
    __shared__ uint32_t cnt[KM_MAX_C];
    const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int32_t* a = assign + (int64_t)h * nq;
    if (tid < C) cnt[tid] = 0u;
    __syncthreads();
    const int64_t p1 = min(nq, (int64_t)(r + 1) * span);
    for (int64_t p = (int64_t)r * span + tid; p < p1; p += 1024) atomicAdd(&cnt[km_centre(a, p, C)], 1u);
    __syncthreads();
    if (tid < C) counts[((int64_t)h * gridDim.x + r) * C + tid] = cnt[tid];
}

__global__ __launch_bounds__(1024) void km_place_kernel(const int32_t* __restrict__ assign, int64_t nq, int C,
                                                        int64_t span, const uint32_t* __restrict__ counts,
                                                        int32_t* __restrict__ perm) {
    __shared__ uint32_t tot[KM_MAX_C], base[KM_MAX_C];
    __shared__ uint32_t wc[16][KM_MAX_C];
    const int r = blockIdx.x, nr = gridDim.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int32_t* a = assign + (int64_t)h * nq;
    int32_t* out = perm + (int64_t)h * nq;
    const uint32_t* ch = counts + (int64_t)h * nr * C;
    if (tid < C) tot[tid] = base[tid] = 0u;
    __syncthreads();
    for (int i = tid; i < nr * C; i += 1024) {       // every centre's total, and its rows in earlier ranges
        const uint32_t v = ch[i];
        atomicAdd(&tot[i % C], v);
        if (i / C < r) atomicAdd(&base[i % C], v);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0u;
        for (int c = 0; c < C; ++c) {
            base[c] += acc;
            acc += tot[c];
        }
    }
    __syncthreads();
    const int64_t p0s = (int64_t)r * span, p1 = min(nq, p0s + span);
    int cn = p0s + tid < p1 ? km_centre(a, p0s + tid, C) : -1;
    for (int64_t p0 = p0s; p0 < p1; p0 += 1024) {
        const int64_t p = p0 + tid;
        const int c = cn;
        cn = p + 1024 < p1 ? km_centre(a, p + 1024, C) : -1;
        // this wave's count of every centre, and each lane's rank among the lanes of its centre:
        // one ballot per distinct centre present (rows that cluster bring few)
        if (lane < C) wc[w][lane] = 0u;
        uint32_t rank = 0u;
        uint64_t todo = __ballot(c >= 0);
        while (todo) {
            const int cc = __builtin_amdgcn_readlane(c, __builtin_ctzll(todo));
            const uint64_t bal = __ballot(c == cc);
            if (lane == 0) wc[w][cc] = (uint32_t)__popcll(bal);
            if (c == cc) rank = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
            todo &= ~bal;
        }
        __syncthreads();
        if (c >= 0) {
            uint32_t pos = base[c] + rank;
            for (int ww = 0; ww < w; ++ww) pos += wc[ww][c];
            out[pos] = (int32_t)p;
        }
        __syncthreads();
        if (tid < C) {
            uint32_t acc = 0u;
            for (int ww = 0; ww < 16; ++ww) acc += wc[ww][tid];
            base[tid] += acc;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// dequant_rows: out[r, :] = e4m3(x8[r, :]) * scale[r] (h3/htrc_flat_triton.py:276-294), the
// per-token fp8 cache to bf16 (or fp32) in one pass.  Rows of x8 and scale may be strided
// views; out is contiguous [rows, d].  One thread per element, consecutive threads on
// consecutive elements of a row.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {   // OCP e4m3fn: bias 7, no infinities
    const uint32_t sgn = (b & 0x80u) << 24, e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15u && m == 7u) return __uint_as_float(sgn | 0x7fc00000u);                    // NaN
    if (e == 0u) return __uint_as_float(sgn | __float_as_uint((float)m * 0.001953125f));   // m * 2^-9
    return __uint_as_float(sgn | ((e + 120u) << 23) | (m << 20));
}

template <bool OUT_BF16>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ x8, int64_t stride_x,
                                                      const float* __restrict__ scale, int64_t stride_s,
                                                      int64_t rows, int d, void* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * d) return;
    const int64_t r = i / d;
    const int c = (int)(i - r * d);
    const float y = __fmul_rn(e4m3_to_f32(x8[r * stride_x + c]), scale[r * stride_s]);
    if (OUT_BF16)
        ((uint16_t*)out)[i] = (uint16_t)f2bf(y);
    else
        ((float*)out)[i] = y;
}

// ---------------------------------------------------------------------------------------------
// bound_select: the reference's alternative routing score (select="bound", h3/htrc_flat.py:255-257;
// the bf16 state store): SEL[t, l] = lz[t, l] + r_t * ||g_tl|| with r_t the largest ||q_row - mu_t||
// over the tile group's rows, padded as the reference pads its tiles (rows past the last query
// repeat it, tiles past the last tile repeat it).  Each norm is a sequential fp32 sum of squares
// over the dims and one IEEE square root.  One workgroup per tile group of the window; padded
// leaves get -inf.  (sqrtf, which HIP keeps correctly rounded by default: the header's __fsqrt_rn
// is the native approximation unless the OCML rounded operations are enabled.)
// ---------------------------------------------------------------------------------------------
template <bool IN_BF16, bool G_F32 = false>
__global__ __launch_bounds__(256) void bound_select_kernel(const void* __restrict__ qin, const float* __restrict__ mu,
                                                           const void* __restrict__ g, const float* __restrict__ lz,
                                                           int64_t nq, int nt, int tile, int group, int ng_all, int g0,
                                                           int gn, int nb, int nb_pad, const int32_t* __restrict__ perm,
                                                           float* __restrict__ sel) {
    __shared__ float smu[D];
    __shared__ float red[256];
    const int gi = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int64_t gs = (int64_t)h * gn + gi;                 // state / SEL row of the window
    const int64_t mrow = (int64_t)h * ng_all + g0 + gi;      // centre of the group
    if (tid < D) smu[tid] = mu[mrow * D + tid];
    __syncthreads();
    const int rows = group * tile;
    const int64_t qbase = (int64_t)h * nq * D;
    float best = 0.0f;                                       // norms are >= 0
    for (int rr = tid; rr < rows; rr += 256) {
        const int t = min((g0 + gi) * group + rr / tile, nt - 1);
        const int64_t pp = min((int64_t)t * tile + rr % tile, nq - 1);
        const int64_t p = perm_row(perm, h, nq, pp);
        float s = 0.0f;
        for (int c = 0; c < D; ++c) {
            const float x = IN_BF16 ? bf2f(((const uint16_t*)qin)[qbase + p * D + c]) : ((const float*)qin)[qbase + p * D + c];
            const float dl = __fsub_rn(x, smu[c]);
            s = __fadd_rn(s, __fmul_rn(dl, dl));
        }
        best = fmaxf(best, sqrtf(s));
    }
    red[tid] = best;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
        __syncthreads();
    }
    const float r = red[0];
    for (int l = tid; l < nb_pad; l += 256) {
        float val = -INFINITY;
        if (l < nb) {
            const int64_t gr = (gs * nb_pad + l) * D;
            float s = 0.0f;
            for (int c = 0; c < D; ++c) {
                const float x = G_F32 ? ((const float*)g)[gr + c] : bf2f(((const uint16_t*)g)[gr + c]);
                s = __fadd_rn(s, __fmul_rn(x, x));
            }
            val = __fadd_rn(lz[gs * nb_pad + l], __fmul_rn(r, sqrtf(s)));
        }
        sel[gs * nb_pad + l] = val;
    }
}

// ---------------------------------------------------------------------------------------------
// fake_quant: the reference's accuracy simulation (h3/htrc_flat.py:68-96): each group of gsz
// consecutive values round-trips through a low-bit format with one symmetric scale s =
// max(max|x|, 1e-20) / qmax of the group: int8 / int4 (qmax 127 / 7): rint(x / s) clamped to
// +-qmax, times s; fp8 (448): the e4m3fn code of x / s clamped to +-448 (nearest even), decoded,
// times s; fp4 (6): the e2m1 magnitude {0, .5, 1, 1.5, 2, 3, 4, 6} chosen by the thresholds
// {.25, .75, 1.25, 1.75, 2.5, 3.5, 5} (a value on a threshold takes the lower magnitude), with
// x's sign, times s.  Divisions and products are single IEEE fp32 operations, as the torch ops
// are.  One thread per group (groups of 16 .. 128 values: two passes over data in cache).
// ---------------------------------------------------------------------------------------------
enum FakeQuantFmt { FQ_INT8 = 0, FQ_INT4 = 1, FQ_FP8 = 2, FQ_FP4 = 3 };

template <bool IN_BF16, bool OUT_BF16>
__global__ __launch_bounds__(256) void fake_quant_kernel(const void* __restrict__ x, int64_t groups, int gsz, int fmt,
                                                         void* __restrict__ out) {
    const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= groups) return;
    const int64_t base = gi * gsz;
    auto ld = [&](int j) {
        return IN_BF16 ? bf2f(((const uint16_t*)x)[base + j]) : ((const float*)x)[base + j];
    };
    float amax = 0.0f;
    for (int j = 0; j < gsz; ++j) amax = fmaxf(amax, fabsf(ld(j)));
    amax = fmaxf(amax, 1e-20f);
    const float qmax = fmt == FQ_INT8 ? 127.0f : fmt == FQ_INT4 ? 7.0f : fmt == FQ_FP8 ? 448.0f : 6.0f;
    const float sc = __fdiv_rn(amax, qmax);
    for (int j = 0; j < gsz; ++j) {
        const float y = ld(j);
        const float t = __fdiv_rn(y, sc);
        float r;
        if (fmt == FQ_INT8 || fmt == FQ_INT4) {
            r = fminf(fmaxf(rintf(t), -qmax), qmax);
        } else if (fmt == FQ_FP8) {
            r = e4m3_to_f32(f32_to_e4m3(fminf(fmaxf(t, -448.0f), 448.0f)));
        } else {
            const float a = fabsf(t);
            const float m = a <= 0.25f ? 0.0f : a <= 0.75f ? 0.5f : a <= 1.25f ? 1.0f : a <= 1.75f ? 1.5f
                          : a <= 2.5f ? 2.0f : a <= 3.5f ? 3.0f : a <= 5.0f ? 4.0f : 6.0f;
            r = y > 0.0f ? m : (y < 0.0f ? -m : 0.0f);
        }
        const float o = __fmul_rn(r, sc);
        if (OUT_BF16)
            ((uint16_t*)out)[base + j] = (uint16_t)f2bf(o);
        else
            ((float*)out)[base + j] = o;
    }
}

__global__ __launch_bounds__(64) void selftest_mfma_kernel(const int8_t* __restrict__ ai, const int8_t* __restrict__ bi,
                                                           int32_t* __restrict__ ci, const uint16_t* __restrict__ af,
                                                           const uint16_t* __restrict__ bf, float* __restrict__ cf) {
    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    i32x4 a = *(const i32x4*)(ai + col * 64 + 16 * grp);
    int8_t bb[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) bb[e] = bi[(16 * grp + e) * 16 + col];
    i32x4 b = __builtin_bit_cast(i32x4, bb);
    i32x4 c = mfma_i8(a, b, i32x4{0, 0, 0, 0});
#pragma unroll
    for (int i = 0; i < 4; ++i) ci[(4 * grp + i) * 16 + col] = c[i];
    const bf16x8 fa = as_bf16x8(*(const u32x4*)(af + col * 32 + 8 * grp));
    uint16_t fb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) fb[e] = bf[(8 * grp + e) * 16 + col];
    const bf16x8 fbv = __builtin_bit_cast(bf16x8, fb);
    f32x4 cc = mfma_bf16(fa, fbv, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int i = 0; i < 4; ++i) cf[(4 * grp + i) * 16 + col] = cc[i];
}

// selftest_f32_e4m3: the stats kernel's fp32 -> e4m3 codes (quant4_e4m3_cvt, c = 1) next to
// f32_to_e4m3, four values per thread.
__global__ __launch_bounds__(64) void selftest_f32_e4m3_kernel(const float* __restrict__ x, int n,
                                                               uint32_t* __restrict__ cvt, uint32_t* __restrict__ soft) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (4 * i >= n) return;
    const f32x4 v = *(const f32x4*)(x + 4 * i);
    cvt[i] = quant4_e4m3_cvt(v, 1.0f);
    soft[i] = quant4_e4m3(v, 1.0f);
}

// selftest_e4m3: the route kernels' e4m3 -> fp16 widening (e4m3x8_to_h8_cvt), eight codes per
// thread, next to the bit-exact field shift (e4m3x8_to_h8).
__global__ __launch_bounds__(64) void selftest_e4m3_kernel(const uint8_t* __restrict__ codes, int n,
                                                           uint16_t* __restrict__ cvt, uint16_t* __restrict__ bits) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (8 * i >= n) return;
    const u32x2 c = *(const u32x2*)(codes + 8 * i);
    *(u32x4*)(cvt + 8 * i) = e4m3x8_to_h8_cvt(c);
    *(u32x4*)(bits + 8 * i) = e4m3x8_to_h8(c);
}

// =============================================================================================
// C-ABI launchers
// =============================================================================================
#include "htrc_flat.h"

// Scratch of htrc_route_noalloc, the route entry point that allocates nothing: rowmax, the near
// leaves and (above ROUTE_NB_LDS leaves per head) the top-k keys live here instead of in caller
// workspace.  Each device that runs the library holds its own copy until the process ends; host
// code reaches it only through the address hipGetSymbolAddress returns on that device.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static thread_local char g_err[512] = "";

static int fail(int code, const char* msg) {
    snprintf(g_err, sizeof(g_err), "%s", msg);
    return code;
}

static int launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof(g_err), "%s: launch failed: %s", what, hipGetErrorString(e));
        return HTRC_ERR_HIP;
    }
    g_err[0] = 0;
    return HTRC_OK;
}

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

#define REQUIRE(cond, msg)                             \
    do {                                               \
        if (!(cond)) return fail(HTRC_ERR_ARG, msg);   \
    } while (0)

extern "C" {

int htrc_abi_version(void) { return HTRC_ABI_VERSION; }

const char* htrc_last_error(void) { return g_err; }

int htrc_nb_pad(int64_t nb) { return (int)((nb + 31) / 32 * 32); }

int htrc_pack_q(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int tile, int group,
                const int32_t* perm, float* mu, int8_t* q8, float* sq, int8_t* dq8, float* sdq, void* stream) {
    REQUIRE(q && mu && q8 && sq && dq8 && sdq, "htrc_pack_q: null pointer");
    REQUIRE(d == D, "htrc_pack_q: head dim must be 128");
    REQUIRE(tile == 32 || tile == 64, "htrc_pack_q: tile must be 32 or 64 rows");
    REQUIRE(heads > 0 && heads <= 65535 && nq > 0, "htrc_pack_q: bad heads / rows");
    REQUIRE(group >= 1 && group <= 1024, "htrc_pack_q: group must be in [1, 1024]");
    REQUIRE(aligned(q, 16) && aligned(q8, 16) && aligned(dq8, 16), "htrc_pack_q: q and the int8 outputs must be 16-byte aligned");
    const int64_t nt = (nq + tile - 1) / tile;
    REQUIRE(nt <= 0x7fffffff, "htrc_pack_q: too many tiles");
    const int64_t ng = (nt + group - 1) / group;
    hipStream_t s = (hipStream_t)stream;
    if (group > 1) {
        const dim3 gg((unsigned)ng, (unsigned)heads);
        if (q_is_bf16)
            hipLaunchKernelGGL(group_centres_kernel<true>, gg, dim3(D), 0, s, q, nq, (int)nt, tile, group, (int)ng,
                               perm, mu);
        else
            hipLaunchKernelGGL(group_centres_kernel<false>, gg, dim3(D), 0, s, q, nq, (int)nt, tile, group, (int)ng,
                               perm, mu);
    }
    dim3 grid((unsigned)nt, (unsigned)heads);
    if (q_is_bf16)
        hipLaunchKernelGGL(pack_q_kernel<true>, grid, dim3(256), 0, s, q, nq, (int)nt, tile, group, (int)ng, perm, mu,
                           q8, sq, dq8, sdq);
    else
        hipLaunchKernelGGL(pack_q_kernel<false>, grid, dim3(256), 0, s, q, nq, (int)nt, tile, group, (int)ng, perm, mu,
                           q8, sq, dq8, sdq);
    return launched("htrc_pack_q");
}

int htrc_pack_k(const uint16_t* k, int64_t heads, int64_t nk, int d, int8_t* k8, float* ks, void* stream) {
    REQUIRE(k && k8 && ks, "htrc_pack_k: null pointer");
    REQUIRE(d == D, "htrc_pack_k: head dim must be 128");
    REQUIRE(heads > 0 && heads <= 65535 && nk > 0 && nk % 16 == 0, "htrc_pack_k: keys must be a positive multiple of 16");
    REQUIRE(aligned(k, 16) && aligned(k8, 16), "htrc_pack_k: k and k8 must be 16-byte aligned");
    dim3 grid((unsigned)((nk + 63) / 64), (unsigned)heads);
    hipLaunchKernelGGL(pack_k_kernel, grid, dim3(256), 0, (hipStream_t)stream, k, nk, k8, ks);
    return launched("htrc_pack_k");
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Shared checks and launch of the three leaf-statistics stores (STORE 0 int8, 1 bf16, 2 fp8).
extern "C++" {
template <int STORE, bool TF32 = false>
static int leaf_stats_launch(const char* who, const float* mu, const uint16_t* mut, const uint16_t* k, const uint16_t* v,
                             int64_t heads,
                             int64_t nt, int64_t c0, int64_t cn, int64_t nk, int leaf, int d, float scale, void* g,
                             float* sg, void* vb, float* sv, float* lz, void* stream) {
    static thread_local char msg[200];
    auto bad = [&](const char* what) {
        snprintf(msg, sizeof msg, "%s: %s", who, what);
        return fail(HTRC_ERR_ARG, msg);
    };
    constexpr bool HAS_SG = STORE == 0 || STORE == 2;
    if (!((mu || mut) && k && v && g && vb && lz && (!HAS_SG || sg) && (STORE != 2 || sv))) return bad("null pointer");
    if (d != D) return bad("head dim must be 128");
    if (!(leaf == 16 || leaf == 32 || leaf == 64 || leaf == 128)) return bad("leaf must be 16/32/64/128");
    if (!(nk > 0 && nk % leaf == 0)) return bad("key count must be a multiple of the leaf size");
    if (!(heads > 0 && heads <= 65535 && nt > 0 && nt <= 0x7fffffff)) return bad("bad heads / centres");
    if (!(c0 >= 0 && cn > 0 && c0 + cn <= nt)) return bad("centre window [c0, c0 + cn) must lie in [0, nt)");
    if (!(aligned(k, 16) && aligned(v, 16) && aligned(g, 16) && aligned(vb, 16) && aligned(lz, 16) && aligned(mut, 16) &&
          (!HAS_SG || aligned(sg, 16)) && (STORE != 2 || aligned(sv, 16))))
        return bad("misaligned buffer");
    const int64_t nb = nk / leaf;
    const int nbp = htrc_nb_pad(nb);
    // leaf-stationary: NL leaves (64 KB of K / V) per workgroup; the centre groups of a head dealt
    // over ncs workgroups when the leaf groups alone give fewer than two workgroups per CU (each
    // wave keeps at least one group of 16 centres)
    const int nl = 65536 / (512 * leaf);
    const int64_t nlg = nbp / nl, ncg = (cn + 15) / 16;
    const int64_t want = 2 * (int64_t)device_cus();
    int64_t ncs = (want + nlg * heads - 1) / (nlg * heads);
    ncs = ncs < 1 ? 1 : (ncs > (ncg + 3) / 4 ? (ncg + 3) / 4 : ncs);
    const int64_t nblocks = ncs * nlg * heads;
    if (nblocks > 0x7fffffff) return bad("too many centres x leaves x heads for one launch");
    const dim3 grid((unsigned)nblocks);
    hipStream_t s = (hipStream_t)stream;
#define STATS_CASE(L)                                                                                            \
    case L:                                                                                                      \
        if (mut)                                                                                                 \
            hipLaunchKernelGGL((stats_ls_kernel<L, STORE, 65536 / (512 * L), TF32, true>), grid, dim3(256), 0, s, mu,  \
                               mut, nt, c0, (int)cn, k, v, nk, (int)nb, nbp, (int)ncs, scale, (int8_t*)g, sg,        \
                               (uint16_t*)vb, sv, lz);                                                             \
        else                                                                                                     \
            hipLaunchKernelGGL((stats_ls_kernel<L, STORE, 65536 / (512 * L), TF32>), grid, dim3(256), 0, s, mu, mut,   \
                               nt, c0, (int)cn, k, v, nk, (int)nb, nbp, (int)ncs, scale, (int8_t*)g, sg,            \
                               (uint16_t*)vb, sv, lz);                                                             \
        break;
    switch (leaf) {
        STATS_CASE(16)
        STATS_CASE(32)
        STATS_CASE(64)
        STATS_CASE(128)
    }
#undef STATS_CASE
    return launched(who);
}
}  // extern "C++"

int htrc_leaf_stats(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                    int64_t cn, int64_t nk, int leaf, int d, float scale, int8_t* g8, float* sg, uint16_t* vb, float* lz,
                    void* stream) {
    return leaf_stats_launch<0>("htrc_leaf_stats", mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g8, sg, vb,
                                nullptr, lz, stream);
}

int htrc_leaf_stats_fp8(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                        int64_t cn, int64_t nk, int leaf, int d, float scale, uint8_t* g, float* sg, uint8_t* vb,
                        float* sv, float* lz, void* stream) {
    return leaf_stats_launch<2>("htrc_leaf_stats_fp8", mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, sg, vb, sv,
                                lz, stream);
}

int htrc_leaf_stats_bf16(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                         int64_t cn, int64_t nk, int leaf, int d, float scale, uint16_t* g, uint16_t* vb, float* lz,
                         void* stream) {
    return leaf_stats_launch<1>("htrc_leaf_stats_bf16", mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, nullptr,
                                vb, nullptr, lz, stream);
}

int htrc_centre_terms(const float* mu, int64_t heads, int64_t nt, int64_t c0, int64_t cn, int d, int tf32,
                      uint16_t* terms, void* stream) {
    REQUIRE(mu && terms, "htrc_centre_terms: null pointer");
    REQUIRE(d == D, "htrc_centre_terms: head dim must be 128");
    REQUIRE(heads > 0 && heads <= 65535 && nt > 0 && c0 >= 0 && cn > 0 && c0 + cn <= nt && cn <= 0x7fffffff,
            "htrc_centre_terms: centre window [c0, c0 + cn) must lie in [0, nt)");
    REQUIRE(aligned(terms, 16), "htrc_centre_terms: terms must be 16-byte aligned");
    const dim3 grid((unsigned)cn, (unsigned)heads);
    if (tf32)
        hipLaunchKernelGGL(centre_terms_kernel<true>, grid, dim3(64), 0, (hipStream_t)stream, mu, nt, c0, (int)cn, terms);
    else
        hipLaunchKernelGGL(centre_terms_kernel<false>, grid, dim3(64), 0, (hipStream_t)stream, mu, nt, c0, (int)cn, terms);
    return launched("htrc_centre_terms");
}

int htrc_leaf_stats_terms(const uint16_t* terms, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t cn,
                          int64_t nk, int leaf, int d, float scale, int store, int tf32, void* g, float* sg, void* vb,
                          float* sv, float* lz, void* stream) {
    const char* who = "htrc_leaf_stats_terms";
    REQUIRE(terms, "htrc_leaf_stats_terms: null terms");
    REQUIRE(store >= 0 && store <= 3, "htrc_leaf_stats_terms: store must be 0 (int8), 1 (bf16), 2 (fp8) or 3 (fp32)");
    switch (store) {
        case 0:
            return tf32 ? leaf_stats_launch<0, true>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, sg,
                                                     vb, nullptr, lz, stream)
                        : leaf_stats_launch<0>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, sg, vb,
                                               nullptr, lz, stream);
        case 2:
            return tf32 ? leaf_stats_launch<2, true>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, sg,
                                                     vb, sv, lz, stream)
                        : leaf_stats_launch<2>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, sg, vb, sv,
                                               lz, stream);
        case 1:
            return tf32 ? leaf_stats_launch<1, true>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g,
                                                     nullptr, vb, nullptr, lz, stream)
                        : leaf_stats_launch<1>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, nullptr,
                                               vb, nullptr, lz, stream);
        default:
            return tf32 ? leaf_stats_launch<3, true>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g,
                                                     nullptr, vb, nullptr, lz, stream)
                        : leaf_stats_launch<3>(who, nullptr, terms, k, v, heads, cn, 0, cn, nk, leaf, d, scale, g, nullptr,
                                               vb, nullptr, lz, stream);
    }
}

int htrc_leaf_stats_f32(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                        int64_t cn, int64_t nk, int leaf, int d, float scale, int state_bf16, int tf32, void* g,
                        void* vb, float* lz, void* stream) {
    const char* who = "htrc_leaf_stats_f32";
    if (state_bf16)
        return tf32 ? leaf_stats_launch<1, true>(who, mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, nullptr, vb,
                                                 nullptr, lz, stream)
                    : leaf_stats_launch<1>(who, mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, nullptr, vb, nullptr,
                                           lz, stream);
    return tf32 ? leaf_stats_launch<3, true>(who, mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, nullptr, vb,
                                             nullptr, lz, stream)
                : leaf_stats_launch<3>(who, mu, nullptr, k, v, heads, nt, c0, cn, nk, leaf, d, scale, g, nullptr, vb, nullptr,
                                       lz, stream);
}

// Window of tile groups [g0, g0 + gn) of a head of nt tiles in groups of `group`: sets ng (all
// groups), tb (first tile) and ntw (tiles of the window); false when the window is empty or
// leaves the head.
static bool group_window(int64_t nt, int group, int64_t g0, int64_t gn, int64_t& ng, int64_t& tb, int64_t& ntw) {
    if (group < 1 || nt <= 0) return false;
    ng = (nt + group - 1) / group;
    if (g0 < 0 || gn <= 0 || g0 + gn > ng) return false;
    tb = g0 * group;
    const int64_t te = (g0 + gn) * group < nt ? (g0 + gn) * group : nt;
    ntw = te - tb;
    return ntw > 0;
}

extern "C++" {
template <int KIND>   // 0: int8 state, 1: bf16 state, 2: fp8 state
static int select_launch(const char* who, const void* dq, const float* sdq, const void* g, const float* sg,
                         const float* lz, int64_t heads, int64_t nt, int64_t nb, int stride, int tile, int group,
                         int64_t g0, int64_t gn, int d, float* sel, void* stream) {
    static thread_local char msg[200];
    auto bad = [&](const char* what) {
        snprintf(msg, sizeof msg, "%s: %s", who, what);
        return fail(HTRC_ERR_ARG, msg);
    };
    if (!(dq && g && lz && sel && (KIND != 0 || sdq) && (KIND == 1 || sg))) return bad("null pointer");
    if (d != D) return bad("head dim must be 128");
    if (!(tile == 32 || tile == 64)) return bad("tile must be 32 or 64 rows");
    if (!(stride >= 1 && stride <= tile && tile % stride == 0)) return bad("stride must divide the tile");
    if (!(group >= 1 && group <= 1024)) return bad("group must be in [1, 1024]");
    if (!(heads > 0 && heads <= 65535 && nt > 0 && nt <= 0x7fffffff && nb > 0 && nb <= 0x7fffffff))
        return bad("bad sizes");
    int64_t ng, tb, ntw;
    if (!group_window(nt, group, g0, gn, ng, tb, ntw)) return bad("group window [g0, g0 + gn) must lie in the head's groups");
    if (KIND != 0 && !(aligned(dq, 16) && aligned(g, 16) && aligned(lz, 16) && (KIND == 1 || aligned(sg, 16))))
        return bad("misaligned buffer");
    const int nbp = htrc_nb_pad(nb);
    const dim3 grid((unsigned)gn, (unsigned)((nb + 255) / 256), (unsigned)heads);
    hipStream_t s = (hipStream_t)stream;
#define SEL_ARGS (int)nt, group, (int)g0, (int)gn, (int)nb, nbp, sel
    if constexpr (KIND == 0) {
        if (tile == 64)
            hipLaunchKernelGGL(select_kernel<4>, grid, dim3(256), 0, s, (const int8_t*)dq, sdq, stride,
                               (const int8_t*)g, sg, lz, SEL_ARGS);
        else
            hipLaunchKernelGGL(select_kernel<2>, grid, dim3(256), 0, s, (const int8_t*)dq, sdq, stride,
                               (const int8_t*)g, sg, lz, SEL_ARGS);
    } else {
        constexpr bool FP8 = KIND == 2;
        if (tile == 64)
            hipLaunchKernelGGL((select16_kernel<FP8, 4>), grid, dim3(256), 0, s, (const uint16_t*)dq, stride, g, sg, lz,
                               SEL_ARGS);
        else
            hipLaunchKernelGGL((select16_kernel<FP8, 2>), grid, dim3(256), 0, s, (const uint16_t*)dq, stride, g, sg, lz,
                               SEL_ARGS);
    }
#undef SEL_ARGS
    return launched(who);
}
}  // extern "C++"

int htrc_select(const int8_t* dq8, const float* sdq, const int8_t* g8, const float* sg, const float* lz,
                int64_t heads, int64_t nt, int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn, int d,
                float* sel, void* stream) {
    return select_launch<0>("htrc_select", dq8, sdq, g8, sg, lz, heads, nt, nb, stride, tile, group, g0, gn, d, sel,
                            stream);
}

int htrc_topk(const float* sel, int64_t rows, int64_t nb, int kx, int sink, int32_t* idx, int8_t* excl,
              void* stream) {
    REQUIRE(sel && idx && excl, "htrc_topk: null pointer");
    REQUIRE(rows > 0 && rows <= 0x7fffffff && nb > 0 && nb <= 0x7fffffff, "htrc_topk: bad rows / leaves");
    REQUIRE(kx > 0 && kx <= nb && sink >= 0, "htrc_topk: need 0 < k <= leaves");
    if (nb <= MAX_NB_LDS)
        hipLaunchKernelGGL(topk_kernel<true>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, sel, (int)nb,
                           htrc_nb_pad(nb), kx, sink, idx, excl);
    else
        hipLaunchKernelGGL(topk_kernel<false>, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, sel, (int)nb,
                           htrc_nb_pad(nb), kx, sink, idx, excl);
    return launched("htrc_topk");
}

static int64_t split_len(int64_t n, int64_t ns, int64_t bn) {   // _split, h3/htrc_flat_triton.py:297-299
    const int64_t per = (n + ns - 1) / ns;
    const int64_t r = (per + bn - 1) / bn * bn;
    return r > bn ? r : bn;
}

extern "C++" {
template <int KIND>   // 0: int8 state, 1: bf16 state, 2: fp8 state
static int tile_launch(const char* who, const void* q, const float* sq, const void* dq, const float* sdq, const void* g,
                       const float* sg, const float* lz, const void* vb, const float* sv, const int8_t* excl,
                       const int32_t* idx, const void* k, const float* ks, const uint16_t* v, int64_t heads, int64_t nq,
                       int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn,
                       const int32_t* perm, int splits, int bn, float scale, float* pm, float* pl, float* pacc,
                       float* out, float* logz, void* stream) {
    static thread_local char msg[200];
    auto bad = [&](const char* what) {
        snprintf(msg, sizeof msg, "%s: %s", who, what);
        return fail(HTRC_ERR_ARG, msg);
    };
    if (!(q && dq && g && lz && vb && excl && k && v && (KIND != 0 || (sq && sdq && ks)) && (KIND == 1 || sg) &&
          (KIND != 2 || sv)))
        return bad("null input pointer");
    if (d != D) return bad("head dim must be 128");
    if (!(tile == 32 || tile == 64)) return bad("tile must be 32 or 64 rows");
    if (!(leaf == 16 || leaf == 32 || leaf == 64 || leaf == 128)) return bad("leaf must be 16/32/64/128");
    if (!(nk > 0 && nk % leaf == 0 && nq > 0 && heads > 0 && heads <= 65535)) return bad("bad sizes");
    const int64_t nb = nk / leaf, nt = (nq + tile - 1) / tile;
    if (!(nt <= 0x7fffffff && nb <= 0x7fffffff)) return bad("too many tiles / leaves");
    if (!(kx >= 0 && kx <= nb && (kx == 0 || idx))) return bad("need 0 <= kx <= leaves and idx when kx > 0");
    if (!(splits >= 1 && splits <= 64 && bn >= 32 && bn % 32 == 0))
        return bad("need 1 <= splits <= 64 and a block that is a multiple of 32");
    if (!(splits == 1 ? (out && logz) : (pm && pl && pacc))) return bad("missing outputs");
    if (!(group >= 1 && group <= 1024)) return bad("group must be in [1, 1024]");
    int64_t ng, tb, ntw;
    if (!group_window(nt, group, g0, gn, ng, tb, ntw)) return bad("group window [g0, g0 + gn) must lie in the head's groups");
    if (KIND != 0 && !(aligned(q, 16) && aligned(dq, 16) && aligned(g, 16) && aligned(k, 16) && aligned(lz, 16) &&
                       (KIND == 1 || aligned(sg, 16)) && (KIND != 2 || aligned(sv, 16))))
        return bad("misaligned buffer");
    const int lps = (int)split_len(nb, splits, bn), eps = (int)split_len((int64_t)kx * leaf, splits, bn);
    const dim3 grid((unsigned)ntw, (unsigned)splits, (unsigned)heads);
    hipStream_t s = (hipStream_t)stream;
    float* ppm = splits == 1 ? nullptr : pm;
    float* ppl = splits == 1 ? nullptr : pl;
    float* ppa = splits == 1 ? nullptr : pacc;
#define TILE_TAIL nq, (int)nt, tile, group, (int)g0, (int)gn, perm, nk, (int)nb, htrc_nb_pad(nb), kx, lps, eps, scale, \
                  ppm, ppl, ppa, out, logz
#define TILE_CASE(L)                                                                                               \
    case L:                                                                                                        \
        if constexpr (KIND == 0)                                                                                   \
            hipLaunchKernelGGL(tile_kernel<L>, grid, dim3(4 * tile), 0, s, (const int8_t*)q, sq, (const int8_t*)dq, sdq, \
                               (const int8_t*)g, sg, lz, (const uint16_t*)vb, excl, idx, (const int8_t*)k, ks, v,   \
                               TILE_TAIL);                                                                         \
        else                                                                                                       \
            hipLaunchKernelGGL((tile16_kernel<L, KIND == 2>), grid, dim3(4 * tile), 0, s, (const uint16_t*)q,         \
                               (const uint16_t*)dq, g, sg, lz, vb, sv, excl, idx, (const uint16_t*)k, v, TILE_TAIL);  \
        break;
    switch (leaf) {
        TILE_CASE(16)
        TILE_CASE(32)
        TILE_CASE(64)
        TILE_CASE(128)
    }
#undef TILE_CASE
#undef TILE_TAIL
    return launched(who);
}
}  // extern "C++"

int htrc_tile(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
              const float* sg, const float* lz, const uint16_t* vb, const int8_t* excl, const int32_t* idx,
              const int8_t* k8, const float* ks, const uint16_t* v, int64_t heads, int64_t nq, int64_t nk,
              int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, int splits,
              int bn, float scale, float* pm, float* pl, float* pacc, float* out, float* logz, void* stream) {
    return tile_launch<0>("htrc_tile", q8, sq, dq8, sdq, g8, sg, lz, vb, nullptr, excl, idx, k8, ks, v, heads, nq, nk,
                          leaf, d, kx, tile, group, g0, gn, perm, splits, bn, scale, pm, pl, pacc, out, logz, stream);
}

// The three template flags of the fp32-dot kernels: q in bf16, state in bf16, TF32 operands.
#define F32_DISPATCH(KERNEL, GRID, BLOCK, ...)                                                                      \
    do {                                                                                                           \
        const int code_ = (q_is_bf16 ? 4 : 0) | (state_bf16 ? 2 : 0) | (tf32 ? 1 : 0);                             \
        switch (code_) {                                                                                           \
            case 0: hipLaunchKernelGGL((KERNEL<false, false, false>), GRID, BLOCK, 0, s, __VA_ARGS__); break;      \
            case 1: hipLaunchKernelGGL((KERNEL<false, false, true>), GRID, BLOCK, 0, s, __VA_ARGS__); break;       \
            case 2: hipLaunchKernelGGL((KERNEL<false, true, false>), GRID, BLOCK, 0, s, __VA_ARGS__); break;       \
            case 3: hipLaunchKernelGGL((KERNEL<false, true, true>), GRID, BLOCK, 0, s, __VA_ARGS__); break;        \
            case 4: hipLaunchKernelGGL((KERNEL<true, false, false>), GRID, BLOCK, 0, s, __VA_ARGS__); break;       \
            case 5: hipLaunchKernelGGL((KERNEL<true, false, true>), GRID, BLOCK, 0, s, __VA_ARGS__); break;        \
            case 6: hipLaunchKernelGGL((KERNEL<true, true, false>), GRID, BLOCK, 0, s, __VA_ARGS__); break;        \
            default: hipLaunchKernelGGL((KERNEL<true, true, true>), GRID, BLOCK, 0, s, __VA_ARGS__); break;        \
        }                                                                                                          \
    } while (0)

int htrc_select_f32(const void* q, int q_is_bf16, const float* mu, const void* g, int state_bf16, const float* lz,
                    int64_t heads, int64_t nq, int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn,
                    const int32_t* perm, int tf32, int d, float* sel, void* stream) {
    REQUIRE(q && mu && g && lz && sel, "htrc_select_f32: null pointer");
    REQUIRE(d == D, "htrc_select_f32: head dim must be 128");
    REQUIRE(tile == 32 || tile == 64, "htrc_select_f32: tile must be 32 or 64 rows");
    REQUIRE(stride >= 1 && tile % stride == 0, "htrc_select_f32: stride must divide the tile");
    REQUIRE(heads > 0 && heads <= 65535 && nq > 0 && nb > 0 && nb <= 0x7fffffff, "htrc_select_f32: bad sizes");
    REQUIRE(group >= 1 && group <= 1024, "htrc_select_f32: group must be in [1, 1024]");
    REQUIRE(aligned(q, 16) && aligned(mu, 16) && aligned(g, 16), "htrc_select_f32: misaligned buffer");
    const int64_t nt = (nq + tile - 1) / tile;
    REQUIRE(nt <= 0x7fffffff, "htrc_select_f32: too many tiles");
    int64_t ng, tb, ntw;
    REQUIRE(group_window(nt, group, g0, gn, ng, tb, ntw), "htrc_select_f32: group window [g0, g0 + gn) must lie in the head's groups");
    REQUIRE(gn <= 65535, "htrc_select_f32: at most 65535 groups per launch");
    const int64_t per = SEL_F32_LPW;                       // leaves per workgroup
    const dim3 grid((unsigned)((nb + per - 1) / per), (unsigned)gn, (unsigned)heads);
    hipStream_t s = (hipStream_t)stream;
    F32_DISPATCH(select_f32_kernel, grid, dim3(256), q, mu, (int)ng, g, lz, nq, (int)nt, tile, stride, group, (int)g0,
                 (int)gn, perm, (int)nb, htrc_nb_pad(nb), sel);
    return launched("htrc_select_f32");
}

int htrc_tile_f32(const void* q, int q_is_bf16, const float* mu, const void* g, int state_bf16, const float* lz,
                  const void* vb, const int8_t* excl, const int32_t* idx, const uint16_t* k, const uint16_t* v,
                  int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0,
                  int64_t gn, const int32_t* perm, int splits, int bn, int tf32, float scale, float* pm, float* pl,
                  float* pacc, float* out, float* logz, void* stream) {
    REQUIRE(q && mu && g && lz && vb && excl && k && v, "htrc_tile_f32: null input pointer");
    REQUIRE(d == D, "htrc_tile_f32: head dim must be 128");
    REQUIRE(tile == 32 || tile == 64, "htrc_tile_f32: tile must be 32 or 64 rows");
    REQUIRE(leaf == 16 || leaf == 32 || leaf == 64 || leaf == 128, "htrc_tile_f32: leaf must be 16/32/64/128");
    REQUIRE(nk > 0 && nk % leaf == 0 && nq > 0 && heads > 0 && heads <= 65535, "htrc_tile_f32: bad sizes");
    const int64_t nb = nk / leaf, nt = (nq + tile - 1) / tile;
    REQUIRE(nt <= 0x7fffffff && nb <= 0x7fffffff, "htrc_tile_f32: too many tiles / leaves");
    REQUIRE(kx >= 0 && kx <= nb && (kx == 0 || idx), "htrc_tile_f32: need 0 <= kx <= leaves and idx when kx > 0");
    REQUIRE(splits >= 1 && splits <= 64 && bn >= 32 && bn % 32 == 0,
            "htrc_tile_f32: need 1 <= splits <= 64 and a block that is a multiple of 32");
    REQUIRE(splits == 1 ? (out && logz) : (pm && pl && pacc), "htrc_tile_f32: missing outputs");
    REQUIRE(group >= 1 && group <= 1024, "htrc_tile_f32: group must be in [1, 1024]");
    REQUIRE(aligned(q, 16) && aligned(mu, 16) && aligned(g, 16) && aligned(vb, 16) && aligned(k, 16) && aligned(v, 16),
            "htrc_tile_f32: misaligned buffer");
    int64_t ng, tb, ntw;
    REQUIRE(group_window(nt, group, g0, gn, ng, tb, ntw), "htrc_tile_f32: group window [g0, g0 + gn) must lie in the head's groups");
    const int lps = (int)split_len(nb, splits, bn), eps = (int)split_len((int64_t)kx * leaf, splits, bn);
    const dim3 grid((unsigned)ntw, (unsigned)splits, (unsigned)heads);
    hipStream_t s = (hipStream_t)stream;
    F32_DISPATCH(tile_f32_kernel, grid, dim3(4 * tile), q, mu, (int)ng, g, lz, vb, excl, idx, k, v, nq, (int)nt, tile,
                 group, (int)g0, (int)gn, perm, nk, leaf, (int)nb, htrc_nb_pad(nb), kx, lps, eps, scale,
                 splits == 1 ? nullptr : pm, splits == 1 ? nullptr : pl, splits == 1 ? nullptr : pacc, out, logz);
    return launched("htrc_tile_f32");
}
#undef F32_DISPATCH

int htrc_pack_q16(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int tile, int group,
                  const int32_t* perm, int dq_fp16, float* mu, uint16_t* q16, uint16_t* dq16, void* stream) {
    REQUIRE(q && mu && q16 && dq16, "htrc_pack_q16: null pointer");
    REQUIRE(d == D, "htrc_pack_q16: head dim must be 128");
    REQUIRE(tile == 32 || tile == 64, "htrc_pack_q16: tile must be 32 or 64 rows");
    REQUIRE(heads > 0 && heads <= 65535 && nq > 0, "htrc_pack_q16: bad heads / rows");
    REQUIRE(group >= 1 && group <= 1024, "htrc_pack_q16: group must be in [1, 1024]");
    REQUIRE(aligned(q, 16) && aligned(q16, 16) && aligned(dq16, 16), "htrc_pack_q16: misaligned buffer");
    const int64_t nt = (nq + tile - 1) / tile;
    REQUIRE(nt <= 0x7fffffff, "htrc_pack_q16: too many tiles");
    const int64_t ng = (nt + group - 1) / group;
    hipStream_t s = (hipStream_t)stream;
    if (group > 1) {
        const dim3 gg((unsigned)ng, (unsigned)heads);
        if (q_is_bf16)
            hipLaunchKernelGGL(group_centres_kernel<true>, gg, dim3(D), 0, s, q, nq, (int)nt, tile, group, (int)ng,
                               perm, mu);
        else
            hipLaunchKernelGGL(group_centres_kernel<false>, gg, dim3(D), 0, s, q, nq, (int)nt, tile, group, (int)ng,
                               perm, mu);
    }
    dim3 grid((unsigned)nt, (unsigned)heads);
    int8_t* a = (int8_t*)q16;
    int8_t* b = (int8_t*)dq16;
#define PACK16(BF, QM)                                                                                          \
    hipLaunchKernelGGL((pack_q_kernel<BF, QM>), grid, dim3(256), 0, s, q, nq, (int)nt, tile, group, (int)ng, perm, \
                       mu, a, nullptr, b, nullptr)
    if (q_is_bf16) {
        if (dq_fp16) PACK16(true, 2); else PACK16(true, 1);
    } else {
        if (dq_fp16) PACK16(false, 2); else PACK16(false, 1);
    }
#undef PACK16
    return launched("htrc_pack_q16");
}

int htrc_select_fp8(const uint16_t* dq16, const uint8_t* g, const float* sg, const float* lz, int64_t heads, int64_t nt,
                    int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn, int d, float* sel,
                    void* stream) {
    return select_launch<2>("htrc_select_fp8", dq16, nullptr, g, sg, lz, heads, nt, nb, stride, tile, group, g0, gn, d,
                            sel, stream);
}

int htrc_select_bf16(const uint16_t* dq16, const uint16_t* g, const float* lz, int64_t heads, int64_t nt, int64_t nb,
                     int stride, int tile, int group, int64_t g0, int64_t gn, int d, float* sel, void* stream) {
    return select_launch<1>("htrc_select_bf16", dq16, nullptr, g, nullptr, lz, heads, nt, nb, stride, tile, group, g0,
                            gn, d, sel, stream);
}

int htrc_tile_fp8(const uint16_t* q16, const uint16_t* dq16, const uint8_t* g, const float* sg, const float* lz,
                  const uint8_t* vb, const float* sv, const int8_t* excl, const int32_t* idx, const uint16_t* k,
                  const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                  int group, int64_t g0, int64_t gn, const int32_t* perm, int splits, int bn, float scale, float* pm,
                  float* pl, float* pacc, float* out, float* logz, void* stream) {
    return tile_launch<2>("htrc_tile_fp8", q16, nullptr, dq16, nullptr, g, sg, lz, vb, sv, excl, idx, k, nullptr, v,
                          heads, nq, nk, leaf, d, kx, tile, group, g0, gn, perm, splits, bn, scale, pm, pl, pacc, out,
                          logz, stream);
}

int htrc_tile_bf16(const uint16_t* q16, const uint16_t* dq16, const uint16_t* g, const float* lz, const uint16_t* vb,
                   const int8_t* excl, const int32_t* idx, const uint16_t* k, const uint16_t* v, int64_t heads,
                   int64_t nq, int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn,
                   const int32_t* perm, int splits, int bn, float scale, float* pm, float* pl, float* pacc, float* out,
                   float* logz, void* stream) {
    return tile_launch<1>("htrc_tile_bf16", q16, nullptr, dq16, nullptr, g, nullptr, lz, vb, nullptr, excl, idx, k,
                          nullptr, v, heads, nq, nk, leaf, d, kx, tile, group, g0, gn, perm, splits, bn, scale, pm, pl,
                          pacc, out, logz, stream);
}

int htrc_merge(const float* pm, const float* pl, const float* pacc, int64_t heads, int64_t nq, int tile, int64_t t0,
               int64_t tn, int splits, int d, const int32_t* perm, float* out, float* logz, void* stream) {
    REQUIRE(pm && pl && pacc && out && logz, "htrc_merge: null pointer");
    REQUIRE(tile == 32 || tile == 64, "htrc_merge: tile must be 32 or 64 rows");
    REQUIRE(d == D && splits >= 1 && heads > 0 && heads <= 65535 && nq > 0, "htrc_merge: bad sizes");
    const int64_t nt = (nq + tile - 1) / tile;
    REQUIRE(nt <= 0x7fffffff, "htrc_merge: too many tiles");
    REQUIRE(t0 >= 0 && tn > 0 && t0 + tn <= nt, "htrc_merge: tile window [t0, t0 + tn) must lie in the head's tiles");
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)tn, (unsigned)heads), dim3(4 * tile), 0, (hipStream_t)stream, pm,
                       pl, pacc, splits, nq, (int)t0, tile, perm, out, logz);
    return launched("htrc_merge");
}

// Shape checks shared by the route entry points; sets nb, nt, ng (all tile groups of a head), tb
// and ntw (first tile and tile count of the window of groups [g0, g0 + gn)) and kxe.
static int route_shapes(const char* who, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                        int group, int64_t g0, int64_t gn, int64_t& nb, int64_t& nt, int64_t& ng, int64_t& tb,
                        int64_t& ntw, int& kxe) {
    static thread_local char msg[200];
    auto bad = [&](const char* what) {
        snprintf(msg, sizeof msg, "%s: %s", who, what);
        return fail(HTRC_ERR_ARG, msg);
    };
    if (d != D) return bad("head dim must be 128");
    if (!(leaf == 16 || leaf == 32 || leaf == 64 || leaf == 128)) return bad("leaf must be 16/32/64/128");
    if (!(tile == 32 || tile == 64)) return bad("tile must be 32 or 64 rows");
    if (!(nk > 0 && nk % leaf == 0 && nq > 0 && heads > 0 && heads <= 65535)) return bad("bad sizes");
    nb = nk / leaf;
    nt = (nq + tile - 1) / tile;
    if (nb > ROUTE_MAX_NB) return bad("at most 262144 leaves per head");
    if (nt > 0x7fffffff) return bad("too many tiles");
    if (kx < 0) return bad("need kx >= 0");
    if (group < 1 || group > 1024) return bad("group must be in [1, 1024]");
    if (!group_window(nt, group, g0, gn, ng, tb, ntw)) return bad("group window [g0, g0 + gn) must lie in the head's groups");
    kxe = (int)(kx < nb ? kx : nb);
    if (kxe > ROUTE_MAX_KX) return bad("at most 8192 near leaves per tile (the split tile kernel takes more)");
    if (ntw * heads > 0x7fffffff || gn * heads > 0x7fffffff) return bad("too many tiles x heads for one launch");
    return HTRC_OK;
}

int htrc_route_select(const int8_t* dq8, const float* sdq, const int8_t* g8, const float* sg, const float* lz,
                      int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink, int stride,
                      int tile, int group, int64_t g0, int64_t gn, int32_t* idx, float* rowmax, uint32_t* keys_ws,
                      void* stream) {
    REQUIRE(dq8 && sdq && g8 && sg && lz && rowmax, "htrc_route_select: null pointer");
    REQUIRE(aligned(g8, 16) && aligned(sg, 16) && aligned(lz, 16), "htrc_route_select: misaligned buffer");
    int64_t nb, nt, ng, tb, ntw;
    int kxe;
    const int rc = route_shapes("htrc_route_select", heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng, tb,
                                ntw, kxe);
    if (rc != HTRC_OK) return rc;
    REQUIRE(sink >= 0, "htrc_route_select: need sink >= 0");
    REQUIRE(kxe == 0 || idx, "htrc_route_select: idx is required when kx > 0");
    REQUIRE(stride >= 1 && stride <= tile && tile % stride == 0, "htrc_route_select: stride must divide the tile");
    const bool gk = nb > ROUTE_NB_LDS;
    REQUIRE(!gk || keys_ws, "htrc_route_select: keys_ws [H, gn, nb_pad] is required above 16384 leaves per head");
    const int nbp = htrc_nb_pad(nb);
    const size_t dyn = gk ? 0 : (size_t)4 * nbp;
#define RSEL(M, N, G)                                                                                           \
    hipLaunchKernelGGL((route_select_kernel<M, N, G>), dim3((unsigned)(gn * heads)), dim3(256), dyn,             \
                       (hipStream_t)stream, dq8, sdq, g8, sg, lz, (int)nt, group, (int)g0, (int)gn, (int)nb, nbp, kxe, \
                       sink, stride, idx, rowmax, keys_ws)
#define RSEL_G(M, N) \
    if (gk) RSEL(M, N, true); else RSEL(M, N, false);
    if (tile == 64) {
        if (group == 1) { RSEL_G(false, 4) } else { RSEL_G(true, 4) }
    } else {
        if (group == 1) { RSEL_G(false, 2) } else { RSEL_G(true, 2) }
    }
#undef RSEL_G
#undef RSEL
    return launched("htrc_route_select");
}

// Dynamic LDS of route_kernel: exclusion bits [nb / 32 + 1] and the tile's near leaves [kxe].
static size_t route_dyn_bytes(int64_t nb, int kxe) { return ((size_t)(nb / 32 + 1) * 4 + (size_t)kxe * 4 + 15) / 16 * 16; }

// Static LDS of route_kernel with NP wave pairs: the ring plus the row reductions.
static size_t route_static_bytes(int np) { return (size_t)np * ROUTE_RS * SLOT_BYTES + 64 * 4 * (1 + np) + 16; }

int htrc_route_attend(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
                      const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
                      const uint16_t* v, const int32_t* idx, const float* rowmax, int64_t heads, int64_t nq,
                      int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn,
                      const int32_t* perm, float scale, float* out, float* logz, void* stream) {
    REQUIRE(q8 && sq && dq8 && sdq && g8 && sg && lz && vb && k8 && ks && v && rowmax && out && logz,
            "htrc_route_attend: null pointer");
    REQUIRE(aligned(vb, 16) && aligned(v, 16) && aligned(g8, 16) && aligned(k8, 16) && aligned(sg, 16) &&
                aligned(ks, 16) && aligned(lz, 16) && aligned(q8, 16) && aligned(dq8, 16),
            "htrc_route_attend: misaligned buffer");
    int64_t nb, nt, ng, tb, ntw;
    int kxe;
    const int rc = route_shapes("htrc_route_attend", heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng, tb,
                                ntw, kxe);
    if (rc != HTRC_OK) return rc;
    REQUIRE(kxe == 0 || idx, "htrc_route_attend: idx is required when kx > 0");
    const int nbp = htrc_nb_pad(nb);
    const dim3 grid((unsigned)(ntw * heads));
    hipStream_t s = (hipStream_t)stream;
    // Wave pairs per tile by the layer's tile count: one (all of the tile's keys; several tiles
    // per CU) when the layer gives every CU at least two tiles, two (key halves merged in LDS)
    // below that, four (key quarters, one tile per CU) when it has no more tiles than CUs; fewer
    // pairs when the near list and exclusion bits would not fit the LDS beside the larger ring.
    // The choice depends on the layer's shape only (not on the window), so repeated calls and
    // every windowing of one layer give identical bits.
    const int64_t cus = device_cus();
    const size_t dyn = route_dyn_bytes(nb, kxe);
    int np = nt * heads >= 2 * cus ? 1 : (nt * heads > cus ? 2 : 4);
    while (np > 1 && route_static_bytes(np) + dyn > ROUTE_LDS_MAX) np /= 2;
    REQUIRE(route_static_bytes(np) + dyn <= ROUTE_LDS_MAX, "htrc_route_attend: near list and exclusion bits exceed the LDS");
#define ROUTE_LAUNCH(L, RB, NP)                                                                                \
    hipLaunchKernelGGL((route_kernel<L, RB, NP, ROUTE_RS>), grid, dim3(128 * NP), dyn, s, q8, sq, dq8, sdq, g8, sg, lz, vb, \
                       k8, ks, v, idx, rowmax, nq, (int)nt, group, (int)g0, (int)gn, perm, nk, (int)nb, nbp, kxe, scale, \
                       out, logz)
#define ROUTE_CASE(L)                                                                                          \
    case L:                                                                                                    \
        if (tile == 64) {                                                                                      \
            if (np == 1) ROUTE_LAUNCH(L, 2, 1);                                                                \
            else if (np == 2) ROUTE_LAUNCH(L, 2, 2);                                                           \
            else ROUTE_LAUNCH(L, 2, 4);                                                                        \
        } else {                                                                                               \
            if (np == 1) ROUTE_LAUNCH(L, 1, 1);                                                                \
            else if (np == 2) ROUTE_LAUNCH(L, 1, 2);                                                           \
            else ROUTE_LAUNCH(L, 1, 4);                                                                        \
        }                                                                                                      \
        break;
    switch (leaf) {
        ROUTE_CASE(16)
        ROUTE_CASE(32)
        ROUTE_CASE(64)
        ROUTE_CASE(128)
    }
#undef ROUTE_CASE
#undef ROUTE_LAUNCH
    return launched("htrc_route_attend");
}

int htrc_route(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
               const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
               const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink,
               int stride, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, float scale, float* out,
               float* logz, int32_t* idx, float* rowmax, uint32_t* keys_ws, void* stream) {
    REQUIRE(q8 && sq && vb && k8 && ks && v && out && logz, "htrc_route: null pointer");
    int rc = htrc_route_select(dq8, sdq, g8, sg, lz, heads, nq, nk, leaf, d, kx, sink, stride, tile, group, g0, gn, idx,
                               rowmax, keys_ws, stream);
    if (rc != HTRC_OK) return rc;
    return htrc_route_attend(q8, sq, dq8, sdq, g8, sg, lz, vb, k8, ks, v, idx, rowmax, heads, nq, nk, leaf, d, kx,
                             tile, group, g0, gn, perm, scale, out, logz, stream);
}

// Shared checks of the 16-bit fused route: route_shapes plus the LDS-held top-k keys.
static int route16_shapes(const char* who, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                          int group, int64_t g0, int64_t gn, int64_t& nb, int64_t& nt, int64_t& ng, int64_t& tb,
                          int64_t& ntw, int& kxe) {
    const int rc = route_shapes(who, heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng, tb, ntw, kxe);
    if (rc != HTRC_OK) return rc;
    if (nb > ROUTE_NB_LDS) {
        static thread_local char msg[160];
        snprintf(msg, sizeof msg, "%s: at most 16384 leaves per head (the split tile path takes more)", who);
        return fail(HTRC_ERR_ARG, msg);
    }
    return HTRC_OK;
}

int htrc_route16_select(const uint16_t* dq16, const void* g, const float* sg, const float* lz, int64_t heads,
                        int64_t nq, int64_t nk, int leaf, int d, int kx, int sink, int stride, int tile, int group,
                        int64_t g0, int64_t gn, int fp8, int32_t* idx, float* rowmax, void* stream) {
    REQUIRE(dq16 && g && lz && rowmax && (!fp8 || sg), "htrc_route16_select: null pointer");
    REQUIRE(aligned(dq16, 16) && aligned(g, 16) && aligned(lz, 16) && (!fp8 || aligned(sg, 16)),
            "htrc_route16_select: misaligned buffer");
    int64_t nb, nt, ng, tb, ntw;
    int kxe;
    const int rc = route16_shapes("htrc_route16_select", heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng,
                                  tb, ntw, kxe);
    if (rc != HTRC_OK) return rc;
    REQUIRE(sink >= 0, "htrc_route16_select: need sink >= 0");
    REQUIRE(kxe == 0 || idx, "htrc_route16_select: idx is required when kx > 0");
    REQUIRE(stride >= 1 && stride <= tile && tile % stride == 0, "htrc_route16_select: stride must divide the tile");
    const int nbp = htrc_nb_pad(nb);
#define RSEL16(F, N)                                                                                             \
    hipLaunchKernelGGL((route_select16_kernel<F, N>), dim3((unsigned)(gn * heads)), dim3(256), (size_t)4 * nbp,   \
                       (hipStream_t)stream, dq16, g, sg, lz, (int)nt, group, (int)g0, (int)gn, (int)nb, nbp, kxe, sink, \
                       stride, idx, rowmax)
    if (tile == 64) {
        if (fp8) RSEL16(true, 4); else RSEL16(false, 4);
    } else {
        if (fp8) RSEL16(true, 2); else RSEL16(false, 2);
    }
#undef RSEL16
    return launched("htrc_route16_select");
}

int htrc_route16_attend(const uint16_t* q16, const uint16_t* dq16, const void* g, const float* sg, const float* lz,
                        const void* vb, const float* sv, const uint16_t* k, const uint16_t* v, const int32_t* idx,
                        const float* rowmax, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                        int group, int64_t g0, int64_t gn, const int32_t* perm, int fp8, float scale, float* out,
                        float* logz, void* stream) {
    REQUIRE(q16 && dq16 && g && lz && vb && k && v && rowmax && out && logz && (!fp8 || (sg && sv)),
            "htrc_route16_attend: null pointer");
    REQUIRE(aligned(q16, 16) && aligned(dq16, 16) && aligned(g, 16) && aligned(vb, 16) && aligned(k, 16) &&
                aligned(v, 16) && aligned(lz, 16) && aligned(out, 16) && (!fp8 || (aligned(sg, 16) && aligned(sv, 16))),
            "htrc_route16_attend: misaligned buffer");
    int64_t nb, nt, ng, tb, ntw;
    int kxe;
    const int rc = route16_shapes("htrc_route16_attend", heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng,
                                  tb, ntw, kxe);
    if (rc != HTRC_OK) return rc;
    REQUIRE(kxe == 0 || idx, "htrc_route16_attend: idx is required when kx > 0");
    const int nbp = htrc_nb_pad(nb);
    const size_t dyn = route_dyn_bytes(nb, kxe);
    const size_t stat = (size_t)2 * R16_SLOT + 64 * 4 + 16;
    REQUIRE(stat + dyn <= ROUTE_LDS_MAX, "htrc_route16_attend: near list and exclusion bits exceed the LDS");
    const dim3 grid((unsigned)(ntw * heads));
    hipStream_t s = (hipStream_t)stream;
#define R16_LAUNCH(L, F, NW, RB)                                                                                  \
    hipLaunchKernelGGL((route16_kernel<L, F, NW, RB>), grid, dim3(64 * NW), dyn, s, q16, dq16, g, sg, lz, vb, sv, k, v, idx, \
                       rowmax, nq, (int)nt, group, (int)g0, (int)gn, perm, nk, (int)nb, nbp, kxe, scale, out, logz)
#define R16_CASE(L)                                                                                               \
    case L:                                                                                                       \
        if (tile == 64) {                                                                                         \
            if (fp8) R16_LAUNCH(L, true, 2, 2); else R16_LAUNCH(L, false, 2, 2);                                  \
        } else {                                                                                                  \
            if (fp8) R16_LAUNCH(L, true, 2, 1); else R16_LAUNCH(L, false, 2, 1);                                  \
        }                                                                                                         \
        break;
    switch (leaf) {
        R16_CASE(16)
        R16_CASE(32)
        R16_CASE(64)
        R16_CASE(128)
    }
#undef R16_CASE
#undef R16_LAUNCH
    return launched("htrc_route16_attend");
}

int htrc_route16(const uint16_t* q16, const uint16_t* dq16, const void* g, const float* sg, const float* lz,
                 const void* vb, const float* sv, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nq,
                 int64_t nk, int leaf, int d, int kx, int sink, int stride, int tile, int group, int64_t g0, int64_t gn,
                 const int32_t* perm, int fp8, float scale, float* out, float* logz, int32_t* idx, float* rowmax,
                 void* stream) {
    int rc = htrc_route16_select(dq16, g, sg, lz, heads, nq, nk, leaf, d, kx, sink, stride, tile, group, g0, gn, fp8,
                                 idx, rowmax, stream);
    if (rc != HTRC_OK) return rc;
    return htrc_route16_attend(q16, dq16, g, sg, lz, vb, sv, k, v, idx, rowmax, heads, nq, nk, leaf, d, kx, tile, group,
                               g0, gn, perm, fp8, scale, out, logz, stream);
}

// Device address of `scratch` on the current device, resolved once per device (with that device
// current) and kept; nullptr with the error set when the runtime cannot resolve it.
static void* scratch_ptr() {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        fail(HTRC_ERR_HIP, "htrc_route_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(g_err, sizeof(g_err), "htrc_route_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                     hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = p;
    }
    return addr[dev];
}

int htrc_route_noalloc(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
                       const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
                       const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink,
                       int stride, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, float scale,
                       float* out, float* logz, void* stream) {
    REQUIRE(q8 && sq && dq8 && sdq && g8 && sg && lz && vb && k8 && ks && v && out && logz,
            "htrc_route_noalloc: null pointer");
    int64_t nb, nt, ng, tb, ntw;
    int kxe;
    const int rc = route_shapes("htrc_route_noalloc", heads, nq, nk, leaf, d, kx, tile, group, g0, gn, nb, nt, ng, tb,
                                ntw, kxe);
    if (rc != HTRC_OK) return rc;
    // rowmax [H, nt * tile] fp32 | idx [H, gn, kxe] int32 | keys [H, gn, nb_pad] uint32, 256-byte aligned parts;
    // every part is written before it is read, so nothing needs clearing between calls
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t b_rowmax = up((size_t)heads * (size_t)nt * (size_t)tile * 4);
    const size_t b_idx = up((size_t)heads * (size_t)gn * (size_t)kxe * 4);
    const size_t b_keys = nb > ROUTE_NB_LDS ? up((size_t)heads * (size_t)gn * (size_t)htrc_nb_pad(nb) * 4) : 0;
    if (b_rowmax + b_idx + b_keys > NOALLOC_SCRATCH_BYTES) {
        snprintf(g_err, sizeof(g_err),
                 "htrc_route_noalloc: this call needs %zu bytes of scratch; the allocation-free route holds %zu "
                 "(use htrc_route with caller workspace, or fewer heads / a smaller window)",
                 b_rowmax + b_idx + b_keys, NOALLOC_SCRATCH_BYTES);
        return HTRC_ERR_ARG;
    }
    unsigned char* base = (unsigned char*)scratch_ptr();
    if (!base) return HTRC_ERR_HIP;
    float* rowmax = (float*)base;
    int32_t* idx = kxe > 0 ? (int32_t*)(base + b_rowmax) : nullptr;
    uint32_t* keys = b_keys ? (uint32_t*)(base + b_rowmax + b_idx) : nullptr;
    return htrc_route(q8, sq, dq8, sdq, g8, sg, lz, vb, k8, ks, v, heads, nq, nk, leaf, d, kx, sink, stride, tile, group,
                      g0, gn, perm, scale, out, logz, idx, rowmax, keys, stream);
}

static int tail_launch(const void* q, int q_is_bf16, const float* tk, const float* tv, int64_t heads, int64_t nq,
                       int64_t ntail, int d, int mode, float scale, float* out, float* logz, void* stream) {
    REQUIRE(q && tk && tv && out && logz, "htrc_tail: null pointer");
    REQUIRE(d == D, "htrc_tail: head dim must be 128");
    REQUIRE(heads > 0 && heads <= 65535 && nq > 0 && ntail > 0 && ntail <= (1 << 24), "htrc_tail: bad sizes");
    REQUIRE(aligned(out, 16), "htrc_tail: out must be 16-byte aligned");
    const int64_t nt = (nq + TILE - 1) / TILE;
    REQUIRE(nt <= 0x7fffffff, "htrc_tail: too many tiles");
    const dim3 grid((unsigned)nt, (unsigned)heads);
#define TAIL(QB, M)                                                                                         \
    hipLaunchKernelGGL((tail_kernel<QB, M>), grid, dim3(256), 0, (hipStream_t)stream, q, tk, tv, nq, (int)ntail, \
                       scale, out, logz)
    if (q_is_bf16) {
        if (mode == 0) TAIL(true, 0); else if (mode == 1) TAIL(true, 1); else TAIL(true, 2);
    } else {
        if (mode == 0) TAIL(false, 0); else if (mode == 1) TAIL(false, 1); else TAIL(false, 2);
    }
#undef TAIL
    return launched("htrc_tail");
}

int htrc_tail(const void* q, int q_is_bf16, const float* tk, const float* tv, int64_t heads, int64_t nq,
              int64_t ntail, int d, float scale, float* out, float* logz, void* stream) {
    return tail_launch(q, q_is_bf16, tk, tv, heads, nq, ntail, d, 0, scale, out, logz, stream);
}

int htrc_tail_f32(const void* q, int q_is_bf16, const float* tk, const float* tv, int64_t heads, int64_t nq,
                  int64_t ntail, int d, int tf32, float scale, float* out, float* logz, void* stream) {
    return tail_launch(q, q_is_bf16, tk, tv, heads, nq, ntail, d, tf32 ? 2 : 1, scale, out, logz, stream);
}

int htrc_kmeans_order(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int clusters, int sample,
                      int iters, float* centres, int32_t* assign, int32_t* perm, void* stream) {
    REQUIRE(q && centres && assign && perm, "htrc_kmeans_order: null pointer");
    REQUIRE(d == D, "htrc_kmeans_order: head dim must be 128");
    REQUIRE(heads > 0 && heads <= 65535 && nq > 0 && nq <= 0x7fffffff, "htrc_kmeans_order: bad heads / rows");
    REQUIRE(clusters >= 1 && clusters <= KM_MAX_C, "htrc_kmeans_order: clusters must be in [1, 64]");
    REQUIRE(sample >= 1 && iters >= 0 && iters <= 1000, "htrc_kmeans_order: need sample >= 1 and 0 <= iters <= 1000");
    REQUIRE(aligned(q, 16) && aligned(centres, 16), "htrc_kmeans_order: q and centres must be 16-byte aligned");
    const int64_t m = sample < nq ? sample : nq;
    REQUIRE(m <= KM_MAX_SAMPLE, "htrc_kmeans_order: at most 16384 sample rows");
    hipStream_t s = (hipStream_t)stream;
    const dim3 gc((unsigned)clusters, (unsigned)heads);
    const dim3 gs((unsigned)((m + 255) / 256), (unsigned)heads), ga((unsigned)((nq + 255) / 256), (unsigned)heads);
#define KM_LAUNCH(BF)                                                                                              \
    hipLaunchKernelGGL(km_init_kernel<BF>, gc, dim3(D), 0, s, q, nq, (int)m, clusters, centres);                 \
    for (int it = 0; it < iters; ++it) {                                                                           \
        hipLaunchKernelGGL(km_assign_kernel<BF>, gs, dim3(256), 0, s, q, nq, m, (int)m, clusters, centres, assign); \
        hipLaunchKernelGGL(km_update_kernel<BF>, gc, dim3(D), 0, s, q, nq, (int)m, clusters, assign, centres);    \
    }                                                                                                              \
    hipLaunchKernelGGL(km_assign_kernel<BF>, ga, dim3(256), 0, s, q, nq, nq, 0, clusters, centres, assign);
    if (q_is_bf16) {
        KM_LAUNCH(true)
    } else {
        KM_LAUNCH(false)
    }
#undef KM_LAUNCH
    // the sort's per-range counts go to the centres workspace, spent once the last assignment
    // has run: at most KM_SORT_RANGES * clusters <= clusters * D words per head
    const int64_t span = km_sort_span(nq), ranges = (nq + span - 1) / span;
    static_assert(KM_SORT_RANGES <= D, "per-range counts must fit the centres workspace");
    uint32_t* counts = (uint32_t*)centres;
    hipLaunchKernelGGL(km_count_kernel, dim3((unsigned)ranges, (unsigned)heads), dim3(1024), 0, s, assign, nq,
                       clusters, span, counts);
    hipLaunchKernelGGL(km_place_kernel, dim3((unsigned)ranges, (unsigned)heads), dim3(1024), 0, s, assign, nq,
                       clusters, span, counts, perm);
    return launched("htrc_kmeans_order");
}

int htrc_dequant_rows(const uint8_t* x8, int64_t stride_x, const float* scale, int64_t stride_s, int64_t rows,
                      int d, void* out, int out_is_bf16, void* stream) {
    REQUIRE(x8 && scale && out, "htrc_dequant_rows: null pointer");
    REQUIRE(rows >= 0 && d > 0 && stride_x >= d && stride_s >= 0, "htrc_dequant_rows: bad sizes or strides");
    REQUIRE(rows * (int64_t)d <= ((int64_t)1 << 40), "htrc_dequant_rows: too many elements");
    if (rows == 0) return HTRC_OK;
    const int64_t nblk = (rows * d + 255) / 256;
    REQUIRE(nblk <= 0x7fffffff, "htrc_dequant_rows: too many elements for one launch");
    if (out_is_bf16)
        hipLaunchKernelGGL(dequant_kernel<true>, dim3((unsigned)nblk), dim3(256), 0, (hipStream_t)stream, x8, stride_x,
                           scale, stride_s, rows, d, out);
    else
        hipLaunchKernelGGL(dequant_kernel<false>, dim3((unsigned)nblk), dim3(256), 0, (hipStream_t)stream, x8,
                           stride_x, scale, stride_s, rows, d, out);
    return launched("htrc_dequant_rows");
}

static int bound_select_launch(const void* q, int q_is_bf16, const float* mu, const void* g, int g_f32, const float* lz,
                               int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int tile, int group, int64_t g0,
                               int64_t gn, const int32_t* perm, float* sel, void* stream) {
    REQUIRE(q && mu && g && lz && sel, "htrc_bound_select: null pointer");
    REQUIRE(d == D, "htrc_bound_select: head dim must be 128");
    REQUIRE(tile == 32 || tile == 64, "htrc_bound_select: tile must be 32 or 64 rows");
    REQUIRE(leaf > 0 && nk > 0 && nk % leaf == 0 && nq > 0 && heads > 0 && heads <= 65535,
            "htrc_bound_select: bad sizes");
    REQUIRE(group >= 1 && group <= 1024, "htrc_bound_select: group must be in [1, 1024]");
    const int64_t nt = (nq + tile - 1) / tile, nb = nk / leaf;
    REQUIRE(nt <= 0x7fffffff && nb <= 0x7fffffff, "htrc_bound_select: too many tiles or leaves");
    int64_t ng, tb, ntw;
    REQUIRE(group_window(nt, group, g0, gn, ng, tb, ntw), "htrc_bound_select: group window [g0, g0 + gn) must lie in the head's groups");
    REQUIRE(gn <= 0x7fffffff, "htrc_bound_select: too many groups");
    const dim3 grid((unsigned)gn, (unsigned)heads);
#define BOUND(QB, GF)                                                                                            \
    hipLaunchKernelGGL((bound_select_kernel<QB, GF>), grid, dim3(256), 0, (hipStream_t)stream, q, mu, g, lz, nq, \
                       (int)nt, tile, group, (int)ng, (int)g0, (int)gn, (int)nb, htrc_nb_pad(nb), perm, sel)
    if (q_is_bf16) {
        if (g_f32) BOUND(true, true); else BOUND(true, false);
    } else {
        if (g_f32) BOUND(false, true); else BOUND(false, false);
    }
#undef BOUND
    return launched("htrc_bound_select");
}

int htrc_bound_select(const void* q, int q_is_bf16, const float* mu, const uint16_t* g, const float* lz, int64_t heads,
                      int64_t nq, int64_t nk, int leaf, int d, int tile, int group, int64_t g0, int64_t gn,
                      const int32_t* perm, float* sel, void* stream) {
    return bound_select_launch(q, q_is_bf16, mu, g, 0, lz, heads, nq, nk, leaf, d, tile, group, g0, gn, perm, sel,
                               stream);
}

int htrc_bound_select_f32(const void* q, int q_is_bf16, const float* mu, const float* g, const float* lz, int64_t heads,
                          int64_t nq, int64_t nk, int leaf, int d, int tile, int group, int64_t g0, int64_t gn,
                          const int32_t* perm, float* sel, void* stream) {
    return bound_select_launch(q, q_is_bf16, mu, g, 1, lz, heads, nq, nk, leaf, d, tile, group, g0, gn, perm, sel,
                               stream);
}

int htrc_fake_quant(const void* x, int x_is_bf16, int64_t rows, int d, int group, int fmt, void* out, int out_is_bf16,
                    void* stream) {
    REQUIRE(x && out, "htrc_fake_quant: null pointer");
    REQUIRE(fmt >= FQ_INT8 && fmt <= FQ_FP4, "htrc_fake_quant: unknown quant format");
    REQUIRE(rows >= 0 && d > 0 && group > 0 && group <= 4096 && d % group == 0,
            "htrc_fake_quant: quant group must divide the feature size");
    REQUIRE(rows * (int64_t)d <= ((int64_t)1 << 40), "htrc_fake_quant: too many elements");
    if (rows == 0) return HTRC_OK;
    const int64_t groups = rows * (d / group);
    const int64_t nblk = (groups + 255) / 256;
    REQUIRE(nblk <= 0x7fffffff, "htrc_fake_quant: too many groups for one launch");
#define FQ_LAUNCH(I, O)                                                                                         \
    hipLaunchKernelGGL((fake_quant_kernel<I, O>), dim3((unsigned)nblk), dim3(256), 0, (hipStream_t)stream, x, groups, \
                       group, fmt, out)
    if (x_is_bf16) {
        if (out_is_bf16) FQ_LAUNCH(true, true); else FQ_LAUNCH(true, false);
    } else {
        if (out_is_bf16) FQ_LAUNCH(false, true); else FQ_LAUNCH(false, false);
    }
#undef FQ_LAUNCH
    return launched("htrc_fake_quant");
}

int htrc_selftest_f32_e4m3(const float* x, int64_t n, uint8_t* cvt, uint8_t* soft, void* stream) {
    REQUIRE(x && cvt && soft, "htrc_selftest_f32_e4m3: null pointer");
    REQUIRE(n > 0 && n % 4 == 0 && n <= (1 << 26), "htrc_selftest_f32_e4m3: n must be a positive multiple of 4");
    REQUIRE(aligned(x, 16) && aligned(cvt, 4) && aligned(soft, 4), "htrc_selftest_f32_e4m3: misaligned buffer");
    hipLaunchKernelGGL(selftest_f32_e4m3_kernel, dim3((unsigned)((n / 4 + 63) / 64)), dim3(64), 0,
                       (hipStream_t)stream, x, (int)n, (uint32_t*)cvt, (uint32_t*)soft);
    return launched("htrc_selftest_f32_e4m3");
}

int htrc_selftest_e4m3(const uint8_t* codes, int64_t n, uint16_t* cvt, uint16_t* bits, void* stream) {
    REQUIRE(codes && cvt && bits, "htrc_selftest_e4m3: null pointer");
    REQUIRE(n > 0 && n % 8 == 0 && n <= (1 << 24), "htrc_selftest_e4m3: n must be a positive multiple of 8");
    REQUIRE(aligned(codes, 8) && aligned(cvt, 16) && aligned(bits, 16), "htrc_selftest_e4m3: misaligned buffer");
    hipLaunchKernelGGL(selftest_e4m3_kernel, dim3((unsigned)((n / 8 + 63) / 64)), dim3(64), 0, (hipStream_t)stream,
                       codes, (int)n, cvt, bits);
    return launched("htrc_selftest_e4m3");
}

int htrc_selftest_mfma(const int8_t* ai, const int8_t* bi, int32_t* ci, const uint16_t* af, const uint16_t* bf,
                       float* cf, void* stream) {
    REQUIRE(ai && bi && ci && af && bf && cf, "htrc_selftest_mfma: null pointer");
    REQUIRE(aligned(ai, 16) && aligned(af, 16), "htrc_selftest_mfma: A operands must be 16-byte aligned");
    hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, ai, bi, ci, af, bf, cf);
    return launched("htrc_selftest_mfma");
}

}  // extern "C"
