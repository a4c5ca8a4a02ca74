/*
 * C ABI of the MI355X (gfx950) flat-HTRC attention library, libhtrc_flat.so.
 *
 * Plain device pointers, sizes and a HIP stream (passed as void*).  No launcher
 * allocates, frees or synchronises, so every call can be captured in a HIP graph.
 * Every launcher validates its arguments on the host and returns HTRC_OK (0) or an
 * HTRC_ERR_* code; htrc_last_error() then holds a message (per host thread).
 *
 * All tensors carry a leading head dimension H and are contiguous:
 *   q        fp32 or bf16 [H, nq, 128]          k, v  bf16 [H, nk, 128]
 *   mu       fp32 [H, ng, 128]                  nt = ceil(nq / T)  (tiles of T = 64 or 32 rows)
 *   q8, dq8  int8 [H, nt*T, 128]                sq, sdq fp32 [H, nt*T]    (padded rows)
 *   k8       int8 [H, nk, 128], ks fp32 [H, nk]
 *   g8       int8 [H, ng, nbp, 128]             nb = nk / leaf, nbp = htrc_nb_pad(nb)
 *   sg, lz   fp32 [H, ng, nbp]                  padded leaves: sg = 0, lz = -inf
 *   vb       bf16 [H, ng, nbp, 128]             leaf value means
 *   sel      fp32 [H, ng, nbp]                  excl int8 [H, ng, nbp]; idx int32 [H, ng, kx]
 *   pm, pl   fp32 [H, nt, splits, T]            pacc fp32 [H, nt, splits, T, 128]
 *   out      fp32 [H, nq, 128]                  logz fp32 [H, nq]
 *   rowmax   fp32 [H, nt*T]                     per-row far-field maximum (route)
 *
 * tile = T, the query rows per tile (one expansion centre each): 64, or 32 (the reference's
 * runner mode "max", h3/htrc_flat_runner.py:52).  Every entry point of one call chain takes
 * the same T.
 *
 * group = G >= 1 consecutive tiles share one expansion centre, one leaf state and one near
 * set (the reference's kern["group"], h3/htrc_flat.py:223-231): ng = ceil(nt / G) centres,
 * the last group padded with repeats of the last tile.  G = 1 is the plain per-tile path.
 *
 * perm (optional, int32 [H, nq]; NULL = identity): the operator works on the queries in the
 * order perm (row p is query perm[p], order="kmeans"); pack_q gathers through it and the
 * entry points that write out / logz scatter back, so out / logz stay in query order.
 *
 * Windows (the reference's tile_chunk loop, h3/htrc_flat.py:236-273): the entry points after
 * pack_q / pack_k work on the centres (tile groups) [g0, g0 + gn) of every head, so a caller
 * bounds the per-(centre, leaf) state by looping over windows.  The packed operands, rowmax,
 * out and logz are indexed by the whole layer; the state (g8, sg, lz, vb, sv), sel, excl, idx and
 * the split partials are the window's own: their row dimension is gn (the window's tiles for
 * the partials).  g0 = 0, gn = ng is the whole layer in one window.
 *
 * Limits: leaf 16, 32, 64 or 128; d = 128; heads <= 65535.  The fused route (htrc_route_*)
 * takes at most 8192 near leaves per tile and 262144 leaves per head, and keeps the top-k keys
 * of up to 16384 leaves per head in LDS (above that it needs keys_ws); the split tile path
 * (htrc_select / htrc_topk / htrc_tile / htrc_merge) takes any near-leaf count.
 * The reference implements the same path as Triton kernels driven from Python;
 * each entry point below names the reference interface it replaces.
 */
#ifndef HTRC_FLAT_H
#define HTRC_FLAT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HTRC_ABI_VERSION 15

#define HTRC_OK 0
#define HTRC_ERR_ARG 1 /* invalid argument: shape, alignment, null pointer, knob */
#define HTRC_ERR_HIP 2 /* the HIP runtime rejected the launch */

/* Diagnostics (no reference counterpart). */
int htrc_abi_version(void);
const char* htrc_last_error(void);
/* Padded leaf count of the per-(tile, leaf) state: nb rounded up to a multiple of 32. */
int htrc_nb_pad(int64_t nb);

/* Centres and the row int8 of q and q - mu.  group 1: mu[t] is the mean of tile t's real rows;
 * group G > 1: mu[g] is the mean of the G * T padded rows of tiles gG.., and q - mu uses the
 * centre of the row's group.
 * Replaces _tiles (h3/htrc_flat.py:142-156), the group centres (:223-229) and the in-kernel
 * Q / dQ quantisation of _tile_kernel and _rowmax_kernel (h3/htrc_flat_triton.py:104-117,
 * 225-233). */
int htrc_pack_q(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int tile, int group,
                const int32_t* perm, float* mu, int8_t* q8, float* sq, int8_t* dq8, float* sdq, void* stream);

/* K int8 pack (round half to even, per-row scale).
 * Replaces the host-side K pack of _flat_triton (h3/htrc_flat.py:213-219). */
int htrc_pack_k(const uint16_t* k, int64_t heads, int64_t nk, int d, int8_t* k8, float* ks, void* stream);

/* Leaf statistics at the centres [c0, c0 + cn) of every head with the int8 store of g; mu holds
 * nt centres per head (ng when tiles are grouped); the state rows are the window's ([H, cn, ...]).
 * g8 codes = trunc(g * (127 / max|g|) +- 0.5) (half away from zero).
 * Replaces leaf_stats / _stats_kernel (h3/htrc_flat_triton.py:329-345, 41-85). */
int htrc_leaf_stats(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                    int64_t cn, int64_t nk, int leaf, int d, float scale, int8_t* g8, float* sg, uint16_t* vb, float* lz,
                    void* stream);

/* The statistics' centre operands computed once per layer window (no reference counterpart: the
 * reference's stats kernel takes mu as a tl.dot operand directly, h3/htrc_flat_triton.py:52-58):
 * terms [H, cn, 264] uint16, per centre row c0 + c the fp16 words hi[128] | lo[128] of mu 2^s
 * (mu rounded to TF32 first when tf32 = 1) and s (int32) with max|mu| 2^s in [2^14, 2^15).
 * htrc_leaf_stats_terms: the leaf statistics of those cn centres, with the results of the
 * htrc_leaf_stats* entries (bit for bit) and without their per-group split of mu; store 0 int8
 * (sg), 1 bf16, 2 fp8 (sg, sv), 3 fp32.  tf32 = 1 (the reference's PREC "tf32", which its
 * leaf_stats applies for every store, h3/htrc_flat.py:243-245): the terms made with tf32 = 1, and
 * the softmax weights rounded to TF32 before their products. */
int htrc_centre_terms(const float* mu, int64_t heads, int64_t nt, int64_t c0, int64_t cn, int d, int tf32,
                      uint16_t* terms, void* stream);
int htrc_leaf_stats_terms(const uint16_t* terms, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t cn,
                          int64_t nk, int leaf, int d, float scale, int store, int tf32, void* g, float* sg, void* vb,
                          float* sv, float* lz, void* stream);

/* Row-max routing score SEL[g, l] over every `stride`-th row of the group's tiles, for the groups
 * [g0, g0 + gn) of every head; nt = tiles per head.
 * Replaces rowmax_select / _rowmax_kernel (h3/htrc_flat_triton.py:315-326, 214-254). */
int htrc_select(const int8_t* dq8, const float* sdq, const int8_t* g8, const float* sg, const float* lz,
                int64_t heads, int64_t nt, int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn, int d,
                float* sel, void* stream);

/* kx largest SEL per row (leaves < sink forced in), idx ascending, exclusion mask; any leaf count
 * (rows of more than 8192 leaves are read from global memory in each radix pass).
 * Replaces torch.topk + excl.scatter_ (h3/htrc_flat.py:262-265). `rows` = H * gn. */
int htrc_topk(const float* sel, int64_t rows, int64_t nb, int kx, int sink, int32_t* idx, int8_t* excl,
              void* stream);

/* Far + near online softmax of every (tile, split) of the tiles of groups [g0, g0 + gn).
 * splits == 1 writes out/logz directly; splits > 1 writes the window's partials pm/pl/pacc
 * ([H, tiles of the window, splits, T]) for htrc_merge.
 * Replaces tile_attention / _tile_kernel (h3/htrc_flat_triton.py:348-391, 88-211). */
int htrc_tile(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
              const float* sg, const float* lz, const uint16_t* vb, const int8_t* excl, const int32_t* idx,
              const int8_t* k8, const float* ks, const uint16_t* v, int64_t heads, int64_t nq, int64_t nk,
              int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, int splits,
              int bn, float scale, float* pm, float* pl, float* pacc, float* out, float* logz, void* stream);

/* Merge of the split partials of tiles [t0, t0 + tn) into normalised rows, plus logz = max +
 * log(sum); the partials are [H, tn, splits, T].
 * Replaces _merge_kernel (h3/htrc_flat_triton.py:257-273, launched at :389-390). */
int htrc_merge(const float* pm, const float* pl, const float* pacc, int64_t heads, int64_t nq, int tile, int64_t t0,
               int64_t tn, int splits, int d, const int32_t* perm, float* out, float* logz, void* stream);

/* Production path, first launch, for the groups [g0, g0 + gn): select -> top-k per tile group
 * with SEL kept in LDS (in keys_ws [H, gn, nb_pad] uint32 above 16384 leaves per head; NULL
 * otherwise), writing the routing idx [H, gn, min(kx, nb)] (ascending; required when kx > 0)
 * and rowmax fp32 [H, nt*T], each row's largest far-field score (the tile's largest when
 * stride > 1).  Leaves < sink are always selected.
 * Replaces rowmax_select + torch.topk of the chunk loop (h3/htrc_flat.py:258-265). */
int htrc_route_select(const int8_t* dq8, const float* sdq, const int8_t* g8, const float* sg, const float* lz,
                      int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink, int stride,
                      int tile, int group, int64_t g0, int64_t gn, int32_t* idx, float* rowmax, uint32_t* keys_ws,
                      void* stream);

/* Production path, second launch: far + near field of every tile in one softmax whose
 * reference is rowmax, merged into normalised out / logz (one split per tile).
 * Replaces tile_attention + _merge_kernel of the chunk loop (h3/htrc_flat.py:266-271). */
int htrc_route_attend(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
                      const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
                      const uint16_t* v, const int32_t* idx, const float* rowmax, int64_t heads, int64_t nq,
                      int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn,
                      const int32_t* perm, float scale, float* out, float* logz, void* stream);

/* Both launches of the production path: htrc_route_select then htrc_route_attend.
 * Replaces the chunk loop body of _flat_triton after leaf_stats (h3/htrc_flat.py:250-271). */
int htrc_route(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
               const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
               const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink,
               int stride, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, float scale, float* out,
               float* logz, int32_t* idx, float* rowmax, uint32_t* keys_ws, void* stream);

/* htrc_route without caller workspace: rowmax, the near leaves and the top-k keys live in a
 * scratch array of 32 MiB that the library keeps on each device (resolved at the first call on
 * a device); the call allocates nothing, so callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc) can run the fused route.  It
 * needs 4 * H * nt * T + 4 * H * gn * min(kx, nb) bytes (+ 4 * H * gn * nb_pad above 16384
 * leaves per head) within 32 MiB and rejects larger calls with HTRC_ERR_ARG.  Every call on one
 * device shares that device's scratch: calls that overlap on one device (several streams or
 * threads) race and must be serialised by the caller.  No counterpart in the reference. */
int htrc_route_noalloc(const int8_t* q8, const float* sq, const int8_t* dq8, const float* sdq, const int8_t* g8,
                       const float* sg, const float* lz, const uint16_t* vb, const int8_t* k8, const float* ks,
                       const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int sink,
                       int stride, int tile, int group, int64_t g0, int64_t gn, const int32_t* perm, float scale,
                       float* out, float* logz, void* stream);

/* Tail keys: tk, tv fp32 [H, ntail, 128] (keys past the last full leaf) attended exactly by
 * every query and merged in place into a finished out / logz (log-sum-exp merge).  Up to 16
 * tail keys are taken with q, k, v and p rounded to bf16, more in fp32, as the reference does.
 * Replaces the tail handling of tile_attention (h3/htrc_flat_triton.py:187-207, 366-388). */
int htrc_tail(const void* q, int q_is_bf16, const float* tk, const float* tv, int64_t heads, int64_t nq,
              int64_t ntail, int d, float scale, float* out, float* logz, void* stream);
/* The same merge for the fp32-dot path (dot other than "bf16"): every tail key in fp32
 * operands, TF32-rounded when tf32 = 1 (h3/htrc_flat_triton.py:198-207 with DOT = 0). */
int htrc_tail_f32(const void* q, int q_is_bf16, const float* tk, const float* tv, int64_t heads, int64_t nq,
                  int64_t ntail, int d, int tf32, float scale, float* out, float* logz, void* stream);

/* fp8 state store (store="fp8"; h3/htrc_flat_triton.py:65-72, 104-108, 132-153, 165-184,
 * 214-254 with FP8 = 1), run in the reference's stage structure (select, top-k, tile, merge):
 *   q16 bf16 [H, nt*T, 128] = bf16(q), dq16 [H, nt*T, 128] = fp16(q - mu) (dq_fp16 = 1) or
 *   bf16(q - mu) (dq_fp16 = 0); g, vb uint8 e4m3fn [H, ng, nbp, 128] = code(x / s) with row
 *   scales sg, sv fp32 [H, ng, nbp] = max(max|x| * fp32(1/448), 1e-30); lz as the int8 path.
 *   select: SEL = max_r (fp16 dq . g) * sg + lz; tile far: (fp16 dq . g) * sg + lz with
 *   PV (p sv)(fp16) . vb; near: (bf16 q . bf16 k) * scale with PV bf16(p) . v.
 * Replace leaf_stats(store=float8_e4m3fn), rowmax_select and tile_attention on that state. */
int htrc_pack_q16(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int tile, int group,
                  const int32_t* perm, int dq_fp16, float* mu, uint16_t* q16, uint16_t* dq16, void* stream);
int htrc_leaf_stats_fp8(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                        int64_t cn, int64_t nk, int leaf, int d, float scale, uint8_t* g, float* sg, uint8_t* vb,
                        float* sv, float* lz, void* stream);
int htrc_select_fp8(const uint16_t* dq16, const uint8_t* g, const float* sg, const float* lz, int64_t heads, int64_t nt,
                    int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn, int d, float* sel,
                    void* stream);
int htrc_tile_fp8(const uint16_t* q16, const uint16_t* dq16, const uint8_t* g, const float* sg, const float* lz,
                  const uint8_t* vb, const float* sv, const int8_t* excl, const int32_t* idx, const uint16_t* k,
                  const uint16_t* v, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                  int group, int64_t g0, int64_t gn, const int32_t* perm, int splits, int bn, float scale, float* pm,
                  float* pl, float* pacc, float* out, float* logz, void* stream);

/* bf16 state store (store="bf16"; DOT = 1 without FP8 / I8 in h3/htrc_flat_triton.py:82-83,
 * 132-153, 165-184, 214-254): g, vb bf16 [H, ng, nbp, 128], no row scales; q16 / dq16 from
 * htrc_pack_q16 with dq_fp16 = 0 (bf16 q - mu).  select: SEL = max_r bf16 dq . g + lz;
 * tile far: bf16 dq . g + lz with PV bf16(p) . vb; near as the fp8 store.
 * Replace leaf_stats(store=bfloat16), rowmax_select and tile_attention on that state. */
int htrc_leaf_stats_bf16(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                         int64_t cn, int64_t nk, int leaf, int d, float scale, uint16_t* g, uint16_t* vb, float* lz,
                         void* stream);
int htrc_select_bf16(const uint16_t* dq16, const uint16_t* g, const float* lz, int64_t heads, int64_t nt, int64_t nb,
                     int stride, int tile, int group, int64_t g0, int64_t gn, int d, float* sel, void* stream);
int htrc_tile_bf16(const uint16_t* q16, const uint16_t* dq16, const uint16_t* g, const float* lz, const uint16_t* vb,
                   const int8_t* excl, const int32_t* idx, const uint16_t* k, const uint16_t* v, int64_t heads,
                   int64_t nq, int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0, int64_t gn,
                   const int32_t* perm, int splits, int bn, float scale, float* pm, float* pl, float* pacc, float* out,
                   float* logz, void* stream);

/* fp32 dots (dot other than "bf16", DOT = 0 in h3/htrc_flat_triton.py:81-83, 138-141, 159-161,
 * 171-174, 184-185, 245-247; the default flat_attention(..., backend="triton") call): the state g,
 * vb fp32 (store="fp32") or bf16 (store="bf16"; state_bf16 = 1) [H, ng, nbp, 128], lz fp32; q fp32
 * or bf16 (q_is_bf16) [H, nq, 128] in query order with the optional row permutation perm, mu the
 * layer's centres [H, ceil(nt / group), 128] (htrc_pack_q16's), k / v bf16.  Every product is an
 * exact product of the fp32 operands with fp32 sums: bf16 MFMA over operands split into bf16 terms
 * that sum to them exactly (g and q - mu in the select and the far scores, the query row and the
 * softmax weights in the near field, vb and the weights in the far PV), except the far PV of IEEE
 * operands on fp32 rows, on the fp32 MFMA (v_mfma_f32_16x16x4_f32); tf32 = 1 (precision="tf32", PREC "tf32") rounds every operand to TF32
 * (to nearest, ties away) first.  Statistics: g = (w K) scale and vb = w V stored as fp32 or as
 * bf16 (the htrc_leaf_stats_bf16 values when tf32 = 0).  select: SEL = max over every stride-th row
 * of (q - mu) . g + lz.  tile far: (q - mu) . g + lz, PV p . vb; near: (q . k) scale, PV p . v;
 * the reference's running-max softmax per block of 16 far leaves and 32 near tokens; splits > 1
 * writes the partials for htrc_merge.  htrc_bound_select_f32: select="bound" on an fp32 g (htrc_bound_select's rule).
 * Replace leaf_stats(store=float32 / bfloat16, prec), rowmax_select(dot=0) and
 * tile_attention(dot=0) (h3/htrc_flat_triton.py:315-391) and the store="fp32" / dot="tf32"
 * dispatch of h3/htrc_flat.py:196-212. */
int htrc_leaf_stats_f32(const float* mu, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nt, int64_t c0,
                        int64_t cn, int64_t nk, int leaf, int d, float scale, int state_bf16, int tf32, void* g,
                        void* vb, float* lz, void* stream);
int htrc_select_f32(const void* q, int q_is_bf16, const float* mu, const void* g, int state_bf16, const float* lz,
                    int64_t heads, int64_t nq, int64_t nb, int stride, int tile, int group, int64_t g0, int64_t gn,
                    const int32_t* perm, int tf32, int d, float* sel, void* stream);
int htrc_tile_f32(const void* q, int q_is_bf16, const float* mu, const void* g, int state_bf16, const float* lz,
                  const void* vb, const int8_t* excl, const int32_t* idx, const uint16_t* k, const uint16_t* v,
                  int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile, int group, int64_t g0,
                  int64_t gn, const int32_t* perm, int splits, int bn, int tf32, float scale, float* pm, float* pl,
                  float* pacc, float* out, float* logz, void* stream);
int htrc_bound_select_f32(const void* q, int q_is_bf16, const float* mu, const float* g, const float* lz, int64_t heads,
                          int64_t nq, int64_t nk, int leaf, int d, int tile, int group, int64_t g0, int64_t gn,
                          const int32_t* perm, float* sel, void* stream);

/* Fused production path of the 16-bit state stores (fp8 = 1: store="fp8", g / vb e4m3 codes with
 * row scales sg / sv; fp8 = 0: store="bf16", g / vb bf16, sg / sv unused), for the groups
 * [g0, g0 + gn): q16 / dq16 from htrc_pack_q16 (dq fp16 for fp8, bf16 for bf16), k / v bf16.
 * First launch (htrc_route16_select): SEL with the arithmetic of htrc_select_fp8 /
 * htrc_select_bf16 (bit-exact) kept in LDS, its kx largest (leaves < sink forced in) into idx
 * [H, gn, min(kx, nb)] ascending, and rowmax fp32 [H, nt*T], each row's largest far-field score.
 * Second launch (htrc_route16_attend): far + near field of every tile in one softmax whose
 * reference is rowmax, normalised into out / logz -- the products of htrc_tile_fp8 /
 * htrc_tile_bf16.  At most 16384 leaves and 8192 near leaves per head (the split tile path takes
 * more).  Replace rowmax_select + torch.topk + tile_attention of the chunk loop for
 * store=float8_e4m3fn / bfloat16 (h3/htrc_flat.py:250-271; h3/htrc_flat_triton.py:65-72,
 * 132-184, 214-254). */
int htrc_route16_select(const uint16_t* dq16, const void* g, const float* sg, const float* lz, int64_t heads,
                        int64_t nq, int64_t nk, int leaf, int d, int kx, int sink, int stride, int tile, int group,
                        int64_t g0, int64_t gn, int fp8, int32_t* idx, float* rowmax, void* stream);
int htrc_route16_attend(const uint16_t* q16, const uint16_t* dq16, const void* g, const float* sg, const float* lz,
                        const void* vb, const float* sv, const uint16_t* k, const uint16_t* v, const int32_t* idx,
                        const float* rowmax, int64_t heads, int64_t nq, int64_t nk, int leaf, int d, int kx, int tile,
                        int group, int64_t g0, int64_t gn, const int32_t* perm, int fp8, float scale, float* out,
                        float* logz, void* stream);
int htrc_route16(const uint16_t* q16, const uint16_t* dq16, const void* g, const float* sg, const float* lz,
                 const void* vb, const float* sv, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t nq,
                 int64_t nk, int leaf, int d, int kx, int sink, int stride, int tile, int group, int64_t g0, int64_t gn,
                 const int32_t* perm, int fp8, float scale, float* out, float* logz, int32_t* idx, float* rowmax,
                 void* stream);

/* k-means query order: perm int32 [H, nq], the queries ordered by their nearest of `clusters`
 * centres (stable), the centres from `iters` Lloyd steps on `sample` evenly spaced queries.
 * Workspace: centres fp32 [H, clusters, 128], assign int32 [H, nq]; on return centres holds
 * the sort's per-range counts, not the centres.  1 <= clusters <= 64, min(sample, nq) <= 16384.
 * Replaces kmeans_order (h3/htrc_flat.py:47-61). */
int htrc_kmeans_order(const void* q, int q_is_bf16, int64_t heads, int64_t nq, int d, int clusters, int sample,
                      int iters, float* centres, int32_t* assign, int32_t* perm, void* stream);

/* fp8 rows to bf16 (out_is_bf16 = 1) or fp32: out[r, :] = e4m3fn(x8[r, :]) * scale[r], rounded
 * to nearest even.  x8 rows are stride_x bytes apart and scale entries stride_s floats apart
 * (strided head views of a per-token cache); out is contiguous [rows, d].
 * Replaces dequant_rows / _dequant_kernel (h3/htrc_flat_triton.py:276-294). */
int htrc_dequant_rows(const uint8_t* x8, int64_t stride_x, const float* scale, int64_t stride_s, int64_t rows,
                      int d, void* out, int out_is_bf16, void* stream);

/* Bound routing score of the bf16 state store (select="bound"): sel[h, gi, l] = lz + r * ||g_l||
 * with r the largest ||q_row - mu|| over the rows of tile group g0 + gi (rows past the last query
 * and tiles past the last tile repeat the last, as the reference pads its tiles); q [H, nq, d] fp32
 * or bf16 (q_is_bf16), in query order, perm (optional) maps operator rows to queries; mu the
 * layer's centres [H, ceil(nt / group), d]; g bf16 [H, gn, nb_pad, d] and lz [H, gn, nb_pad] the
 * window's state; sel [H, gn, nb_pad] (padded leaves -inf).  Norms: sequential fp32 sums of squares,
 * one IEEE square root.  Replaces the select == "bound" branch of the chunk loop
 * (h3/htrc_flat.py:255-257). */
int htrc_bound_select(const void* q, int q_is_bf16, const float* mu, const uint16_t* g, const float* lz, int64_t heads,
                      int64_t nq, int64_t nk, int leaf, int d, int tile, int group, int64_t g0, int64_t gn,
                      const int32_t* perm, float* sel, void* stream);

/* Fake quantisation (accuracy simulation): out = x round-tripped through a low-bit format with one
 * symmetric scale per group of `group` consecutive values of each row (d % group == 0): fmt 0 int8,
 * 1 int4 (round to nearest even, clamp), 2 fp8 e4m3fn (nearest even), 3 fp4 e2m1 (threshold
 * table, ties to the lower magnitude); x and out are contiguous [rows, d] fp32 or bf16 (x_is_bf16,
 * out_is_bf16; out may alias x).  Replaces fake_quant (h3/htrc_flat.py:68-96). */
int htrc_fake_quant(const void* x, int x_is_bf16, int64_t rows, int d, int group, int fmt, void* out, int out_is_bf16,
                    void* stream);

/* Self-test of the MFMA operand conventions the kernels rely on (no reference counterpart):
 * one 64-lane wave computes C = A B for A int8 [16, 64] / B int8 [64, 16] (i8 path) and
 * A bf16 [16, 32] / B bf16 [32, 16] (bf16 path), loading operands the way the kernels do.
 * ci int32 [16, 16], cf fp32 [16, 16], device pointers. */
int htrc_selftest_mfma(const int8_t* ai, const int8_t* bi, int32_t* ci, const uint16_t* af, const uint16_t* bf,
                       float* cf, void* stream);

/* Self-test of the e4m3 -> fp16 widening of the 16-bit route kernels (no reference counterpart):
 * the n codes (n a multiple of 8) widened to fp16 holding value * 2^-8 by the conversion
 * instruction the kernels use (cvt) and by the exact exponent / mantissa field shift (bits);
 * device pointers. */
int htrc_selftest_e4m3(const uint8_t* codes, int64_t n, uint16_t* cvt, uint16_t* bits, void* stream);

/* Self-test of the fp32 -> e4m3 codes of the fp8 state store (no reference counterpart): the n
 * values (n a multiple of 4) converted by the conversion instruction the stats kernel uses (cvt)
 * and by the exact software rounding (soft, nearest even, |x| saturated at 448); device pointers. */
int htrc_selftest_f32_e4m3(const float* x, int64_t n, uint8_t* cvt, uint8_t* soft, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HTRC_FLAT_H */
