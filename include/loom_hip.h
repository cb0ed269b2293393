/*
 * loom_hip.h -- C ABI of the MI355X (gfx950) backend for the six loom-dataflow
 * example kernels.
 *
 * One entry point per kernel, named after the MLIR function it implements and
 * taking that function's tensors in the same order.  Tensors are plain device
 * pointers to contiguous row-major buffers with the reference's layouts; bf16
 * tensors hold raw bf16 bits, fp32 tensors IEEE floats.  Extents are explicit.
 * The tile_* arguments are the loom.sym block sizes the staged-ETG solver
 * binds (the `__tile_*` suffix of a materialized variant); each entry point
 * validates them and documents how it maps them onto the GPU.  As in the
 * reference, every tile is bounded by the extent of the loop it tiles (the
 * symbol's upper_bound, exported as natural_ub by
 * lib/passes/lcs/src/staged_etg_builder.cpp:1420-1430): a larger value is
 * rejected with LOOM_HIP_EINVAL.  A symbol that a kernel maps onto a
 * workgroup tile takes any multiple of 16 (the MFMA tile edge; the gfx950
 * counterpart of lib/passes/lcs/src/hw_alignment.cpp:16) up to its extent, or
 * the extent itself, and runs on the smallest workgroup tile built for it
 * that covers the value (the largest built tile above them all); other values
 * are LOOM_HIP_EINVAL.  No result depends on that choice.
 *
 * Conventions shared by every entry point:
 *   - `stream` is a hipStream_t (NULL = the default stream); work is only
 *     enqueued, nothing synchronises.
 *   - Return 0 on success; otherwise nonzero (1 = invalid argument,
 *     2 = configuration not built for gfx950, 3 = HIP runtime error) with a
 *     NUL-terminated message in err[0..errlen).  Nothing throws.
 *   - The library never allocates per call and never frees caller memory;
 *     kernels that gather partial results take a caller-owned workspace whose
 *     size the matching *_workspace_bytes function returns.
 *   - Calls are re-entrant; calls on different streams do not share state.
 *
 * Reference boundary replaced: the reference lowers these functions for a
 * Tenstorrent backend after materialization
 * (lib/pipeline/src/loom_materialization_pipeline.cpp:307-313, marked as
 * the place to gate on a backend at :309-310); this library is what a
 * gfx950 backend launches instead of those passes' output.
 */
#ifndef LOOM_HIP_H
#define LOOM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes of every entry point. */
#define LOOM_HIP_OK 0
#define LOOM_HIP_EINVAL 1 /* shapes, tiles, pointers, JSON or workspace rejected */
#define LOOM_HIP_EUNSUP 2 /* legal in the reference, not built for gfx950 */
#define LOOM_HIP_EHIP 3   /* HIP runtime error */

/* Slots of the tiles[] array loom_hip_parse_variant fills (-1 = unbound). */
#define LOOM_HIP_TILE_B 0
#define LOOM_HIP_TILE_M 1
#define LOOM_HIP_TILE_N 2
#define LOOM_HIP_TILE_K 3
#define LOOM_HIP_TILE_S 4
#define LOOM_HIP_TILE_H 5
#define LOOM_HIP_TILE_C 6
#define LOOM_HIP_NTILES 7

/* Library version string ("loom_hip <major>.<minor>.<patch> gfx950").
 * Counterpart of the pybind module's __version__
 * (lib/pipeline/src/loom_pybind.cpp:17-20). */
const char* loom_hip_version(void);

/* @matmul -- examples/mm/IR/00_from_helion_frontend.mlir:2
 *   (x: memref<MxK>, y: memref<KxN>, out: memref<MxN>)
 * out = x . y, bf16 in, fp32 accumulate, bf16 out.
 * (tile_m, tile_n), each a multiple of 16 or its whole extent (tile_m <= M,
 * tile_n <= N), runs as the smallest square workgroup output tile of (64,64),
 * (128,128), (256,256) covering both.  tile_k (1 <= tile_k <= K) is the K step of
 * the reference loop; the kernel stages K in its own LDS steps (the result
 * does not depend on it). */
int loom_hip_matmul(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                    int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                    size_t errlen);

/* @batch_matmul -- examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4
 *   (arg0: memref<BxMxK>, arg1: memref<BxKxN>, arg2: memref<BxMxN>)
 * arg2[b] = arg0[b] . arg1[b].  Tiles as for loom_hip_matmul; tile_b
 * (1 <= tile_b <= B) groups batches in the reference grid and does not
 * change the result. */
int loom_hip_batch_matmul(const void* arg0, const void* arg1, void* arg2, int64_t B, int64_t M,
                          int64_t N, int64_t K, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                          int64_t tile_k, void* stream, char* err, size_t errlen);

/* Bytes of the fp32 partial stack [S, M, N], S = ceil(K / tile_k), that
 * loom_hip_split_k_matmul_gather gathers into (the loom.gather target of
 * examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:30-33). */
size_t loom_hip_split_k_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t tile_k);

/* @split_k_matmul_gather -- examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2
 *   (a: memref<MxK>, b: memref<KxN>, out: memref<MxN>)
 * partials[s] = a[:, s*tile_k : (s+1)*tile_k] . b[s*tile_k : (s+1)*tile_k, :]
 * in fp32 (slab s at gather index s), then out = bf16(sum_s partials[s]) in
 * ascending s.  On return `partials` holds the gathered stack.  tile_k
 * (1 <= tile_k <= K) fixes the slabs; (tile_m, tile_n) as for matmul. */
int loom_hip_split_k_matmul_gather(const void* a, const void* b, void* out, void* partials,
                                   size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                   int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
                                   char* err, size_t errlen);

/* @attention -- examples/flashattn/IR/00_from_helion_frontend.mlir:4
 *   (k: memref<BHxDxSkv>, v: memref<BHxSkvxD>, q: memref<BHxSqxD>, out: memref<BHxSqxD>)
 * Flash-attention forward with online softmax; `scale` multiplies q.k (the
 * reference hard-codes the f16 constant 0.08837890625 at :10); `causal`
 * (not in the reference; needs Sq == Skv) hides key j from query i < j.
 * tile_m (a multiple of 16 up to Sq, or Sq) runs as the smallest workgroup
 * query tile of 64, 128, 192, 256 covering it; tile_b (<= BH) and tile_n (<= Skv, the
 * online-softmax step) are validated, the kernel streams KV in 64-key LDS
 * blocks.  D a multiple of 8 up to 256 (built for 64, 128 and 256; a
 * narrower D runs on the next one up with its padding rows zero; above 128
 * the query tiles are 64 or 128); any Sq and Skv (Skv
 * not a multiple of 8 stages K through registers instead of 16-byte LDS DMA,
 * and k then needs only 2-byte alignment). */
int loom_hip_attention(const void* k, const void* v, const void* q, void* out, int64_t BH,
                       int64_t Sq, int64_t Skv, int64_t D, float scale, int causal,
                       int64_t tile_b, int64_t tile_m, int64_t tile_n, void* stream, char* err,
                       size_t errlen);

/* Bytes of loom_hip_flash_decode's workspace, the gathered split-KV
 * partials (examples/mqa_decode/IR/00_from_helion_frontend.mlir:139-146):
 * lse [ns, B, H] fp32 at offset 0, then o [ns, B, H, D] fp32 at offset
 * align256(ns*B*H*4); ns = ceil(S / tile_s). */
size_t loom_hip_flash_decode_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t S,
                                             int64_t tile_s);

/* @flash_decode -- examples/mqa_decode/IR/00_from_helion_frontend.mlir:6
 *   (k: memref<BxDxS>, v: memref<BxSxD>, q: memref<BxHxD>, out: memref<BxHxD>)
 * H query heads share one KV head.  Split s covers keys
 * [s*tile_s, (s+1)*tile_s); its (lse_s, o_s) land in the workspace, then a
 * second kernel performs the split-0 combine into out.  tile_b (<= B) and
 * tile_n (<= S) are validated and do not change the result.  D a multiple
 * of 8 up to 256 (built for 64, 128 and 256, a narrower D runs on the next
 * one up); any S;
 * any H (a workgroup serves up to 32 query heads, more heads take more
 * workgroups, each streaming the split's K and V).  scale must be finite and
 * positive (the running max is taken over raw scores before scaling). */
int loom_hip_flash_decode(const void* k, const void* v, const void* q, void* out,
                          void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                          int64_t D, int64_t S, float scale, int64_t tile_b, int64_t tile_s,
                          int64_t tile_n, void* stream, char* err, size_t errlen);

/* loom_hip_flash_decode without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  The split partials go to a static device array of 16 MiB
 * (16777216 bytes; each device holds its own copy until the process ends),
 * so loom_hip_flash_decode_workspace_bytes(B, H, D, S, tile_s) must not
 * exceed it -- larger calls return LOOM_HIP_EINVAL (use a larger tile_s, or
 * loom_hip_flash_decode).  Nothing is allocated and no allocating routine is
 * called.  Every call on a device shares that device's array: calls that
 * overlap in time on one device (different streams, concurrent threads)
 * race and must be ordered by the caller.  The first call on each device
 * looks up the array's device address and must be made outside HIP graph
 * capture: made on a stream being captured it returns LOOM_HIP_EINVAL and
 * records nothing; every later call may be captured.  bf16 only; arguments,
 * validation and results otherwise as loom_hip_flash_decode. */
int loom_hip_flash_decode_noalloc(const void* k, const void* v, const void* q, void* out,
                                  int64_t B, int64_t H, int64_t D, int64_t S, float scale,
                                  int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                  char* err, size_t errlen);

/* @helion_mamba2_chunk_scan_kernel -- examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4
 *   (cb: [b,c,G,Q,Q] bf16, x: [b,H,L,P] bf16, dt: [b,H,c,Q] fp32,
 *    dA_cumsum: [b,H,c,Q] fp32, C: [b,G,L,N] bf16, D: [H] fp32,
 *    prev_states_T: [b,c,H,N,P] fp32, out: [b,H,L,P] bf16), L = c*Q.
 * Mamba-2 SSD chunk scan with the intra-chunk causal mask k <= m.
 * tile_b = tile_h = tile_c = 1 (the reference's size-1 subviews skip work
 * otherwise); tile_m (a multiple of 16 up to Q, or Q) runs as the smallest
 * of 64, 128, 192, 256 rows covering it and tile_n (a multiple of 16 up to
 * P, or P) as the smallest of 16, 32, 64 columns covering it (64 above);
 * tile_k (1 <= tile_k <= max(8192, Q), 8192 being the example's loom.sym
 * upper_bound) is the reference's k step and does not change the result.
 * Q <= 512, N <= 256, Q, N, P multiples of 8 (above Q 256 or N 128 a
 * 4-wave build with one workgroup per CU runs it). */
int loom_hip_helion_mamba2_chunk_scan_kernel(
    const void* cb, const void* x, const void* dt, const void* dA_cumsum, const void* C,
    const void* D, const void* prev_states_T, void* out, int64_t batch, int64_t nchunks,
    int64_t nheads, int64_t ngroups, int64_t chunk_size, int64_t headdim, int64_t dstate,
    int64_t tile_b, int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, void* stream, char* err, size_t errlen);

/* ---- f16 variants ----------------------------------------------------------
 * The reference's example IR is f16 throughout (EX(*,00) signatures: f16
 * memrefs).  Each entry point below is its bf16 namesake above with every
 * 16-bit tensor (inputs and outputs alike) in IEEE binary16 instead: same
 * arguments, tiles, workspaces, validation and return codes; MFMAs run on
 * f16 operands (v_mfma_f32_16x16x32_f16) with fp32 accumulation, and every
 * rounding to f16 is to nearest even.  The split-K partials and the decode
 * workspace stay fp32.  loom_hip_helion_mamba2_chunk_scan_kernel_f16 takes
 * the reference's exact signature: every tensor f16, dt, dA_cumsum, D and
 * prev_states_T included (examples/mamba_chunk_scan/IR/
 * 00_from_helion_frontend.mlir:4; widened to fp32 exactly on load). */
int loom_hip_matmul_f16(const void* x, const void* y, void* out, int64_t M, int64_t N, int64_t K,
                        int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream, char* err,
                        size_t errlen);
int loom_hip_batch_matmul_f16(const void* arg0, const void* arg1, void* arg2, int64_t B,
                              int64_t M, int64_t N, int64_t K, int64_t tile_b, int64_t tile_m,
                              int64_t tile_n, int64_t tile_k, void* stream, char* err,
                              size_t errlen);
int loom_hip_split_k_matmul_gather_f16(const void* a, const void* b, void* out, void* partials,
                                       size_t partials_bytes, int64_t M, int64_t N, int64_t K,
                                       int64_t tile_m, int64_t tile_n, int64_t tile_k,
                                       void* stream, char* err, size_t errlen);
int loom_hip_attention_f16(const void* k, const void* v, const void* q, void* out, int64_t BH,
                           int64_t Sq, int64_t Skv, int64_t D, float scale, int causal,
                           int64_t tile_b, int64_t tile_m, int64_t tile_n, void* stream,
                           char* err, size_t errlen);
int loom_hip_flash_decode_f16(const void* k, const void* v, const void* q, void* out,
                              void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                              int64_t D, int64_t S, float scale, int64_t tile_b, int64_t tile_s,
                              int64_t tile_n, void* stream, char* err, size_t errlen);
int loom_hip_helion_mamba2_chunk_scan_kernel_f16(
    const void* cb, const void* x, const void* dt, const void* dA_cumsum, const void* C,
    const void* D, const void* prev_states_T, void* out, int64_t batch, int64_t nchunks,
    int64_t nheads, int64_t ngroups, int64_t chunk_size, int64_t headdim, int64_t dstate,
    int64_t tile_b, int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, void* stream, char* err, size_t errlen);

/* ---- Mamba-2 SSD prologue --------------------------------------------------
 * The chunk-scan example takes cb, dA_cumsum and prev_states_T ready-made
 * (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4); the
 * reference repository has no code that produces them.  These entry points
 * compute them on the GPU from raw Mamba-2 inputs, following the chunked SSD
 * algorithm (Dao & Gu 2024): x [b,H,L,P] bf16, dt [b,H,L] fp32 (after
 * softplus; the same memory as chunk_scan's dt [b,H,c,Q]), A [H] fp32,
 * B and C [b,G,L,N] bf16, L = nchunks * chunk_size, head h reads group
 * h / (H / G).  chunk_size, headdim and dstate are multiples of 16,
 * chunk_size <= 512, headdim <= 256, dstate <= 256 (a multiple of 32 above
 * 32).  The dt, dA_cumsum and prev_states_T of these stages are fp32 in
 * both forms. */

/* dA_cumsum[b,h,c,q] = sum_{q' <= q} dt[b,h,c*Q+q'] * A[h] (fp32; a wave
 * prefix scan, so the summation order differs from a serial loop). */
int loom_hip_ssd_chunk_cumsum(const void* dt, const void* A, void* dA_cumsum, int64_t batch,
                              int64_t nchunks, int64_t nheads, int64_t chunk_size, void* stream,
                              char* err, size_t errlen);

/* cb[b,c,g,i,j] = bf16(sum_n C[b,g,cQ+i,n] B[b,g,cQ+j,n]) for j <= i, else 0. */
int loom_hip_ssd_bmm_chunk(const void* B, const void* C, void* cb, int64_t batch, int64_t nchunks,
                           int64_t ngroups, int64_t chunk_size, int64_t dstate, void* stream,
                           char* err, size_t errlen);

/* prev_states_T [b,c,H,N,P] fp32: zero for c = 0, then
 * prev(c) = exp(dA[c-1,Q-1]) prev(c-1) + sum_k B[k,n] exp(dA[c-1,Q-1] - dA[c-1,k]) dt[c-1,k] x[k,p]
 * over the keys k of chunk c-1 (chunk states and state passing fused). */
int loom_hip_ssd_chunk_state_passing(const void* x, const void* dt, const void* dA_cumsum,
                                     const void* B, void* prev_states_T, int64_t batch,
                                     int64_t nchunks, int64_t nheads, int64_t ngroups,
                                     int64_t chunk_size, int64_t headdim, int64_t dstate,
                                     void* stream, char* err, size_t errlen);

/* All three stages in stream order: dA_cumsum and cb (independent of each
 * other) in one launch, then prev_states_T; the outputs equal those of the
 * three stage entry points above called in turn.  Every stage's checks run
 * before the first launch: a rejected call enqueues nothing. */
int loom_hip_ssd_prologue(const void* x, const void* dt, const void* A, const void* B,
                          const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                          int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                          int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                          char* err, size_t errlen);

/* f16 forms of the SSD stages whose tensors are 16-bit (x, B, C, cb). */
int loom_hip_ssd_bmm_chunk_f16(const void* B, const void* C, void* cb, int64_t batch,
                               int64_t nchunks, int64_t ngroups, int64_t chunk_size,
                               int64_t dstate, void* stream, char* err, size_t errlen);
int loom_hip_ssd_chunk_state_passing_f16(const void* x, const void* dt, const void* dA_cumsum,
                                         const void* B, void* prev_states_T, int64_t batch,
                                         int64_t nchunks, int64_t nheads, int64_t ngroups,
                                         int64_t chunk_size, int64_t headdim, int64_t dstate,
                                         void* stream, char* err, size_t errlen);
int loom_hip_ssd_prologue_f16(const void* x, const void* dt, const void* A, const void* B,
                              const void* C, void* dA_cumsum, void* cb, void* prev_states_T,
                              int64_t batch, int64_t nchunks, int64_t nheads, int64_t ngroups,
                              int64_t chunk_size, int64_t headdim, int64_t dstate, void* stream,
                              char* err, size_t errlen);

/* ---- MLIR memref descriptors ---------------------------------------------
 * A materialized variant is an MLIR function over memrefs; a caller lowered
 * through MLIR's C interface (`_mlir_ciface_<func>`, whose arguments are
 * pointers to ranked descriptors -- StridedMemRefType<T, R> of MLIR's C
 * runner utilities) holds exactly these structs: the allocated and aligned
 * base pointers, the element offset, and sizes and strides in elements.
 * The loom_hip_ciface_* entry points take them in the MLIR function's
 * argument order (extents come from the sizes; the data pointer is
 * aligned + offset elements) and launch the same kernels as the pointer
 * entry points above.  Every argument must be row-major contiguous:
 * innermost stride 1 and each outer stride the product of the sizes inside
 * it (a dimension of size 1 is never stepped over, so its stride is free);
 * other layouts, sizes that disagree between arguments, a null aligned
 * pointer or a negative offset return LOOM_HIP_EINVAL with a message naming
 * the argument.  Element types: 16-bit tensors bf16 (f16 in the _f16 forms);
 * mamba's dt, dA_cumsum, D and prev_states_T fp32 (f16 in the _f16 form). */
typedef struct loom_memref1 { void* allocated; void* aligned; int64_t offset; int64_t sizes[1]; int64_t strides[1]; } loom_memref1_t;
typedef struct loom_memref2 { void* allocated; void* aligned; int64_t offset; int64_t sizes[2]; int64_t strides[2]; } loom_memref2_t;
typedef struct loom_memref3 { void* allocated; void* aligned; int64_t offset; int64_t sizes[3]; int64_t strides[3]; } loom_memref3_t;
typedef struct loom_memref4 { void* allocated; void* aligned; int64_t offset; int64_t sizes[4]; int64_t strides[4]; } loom_memref4_t;
typedef struct loom_memref5 { void* allocated; void* aligned; int64_t offset; int64_t sizes[5]; int64_t strides[5]; } loom_memref5_t;

/* @matmul (x, y, out) -- examples/mm/IR/00_from_helion_frontend.mlir:2 */
int loom_hip_ciface_matmul(const loom_memref2_t* x, const loom_memref2_t* y,
                           const loom_memref2_t* out, int64_t tile_m, int64_t tile_n,
                           int64_t tile_k, void* stream, char* err, size_t errlen);
int loom_hip_ciface_matmul_f16(const loom_memref2_t* x, const loom_memref2_t* y,
                               const loom_memref2_t* out, int64_t tile_m, int64_t tile_n,
                               int64_t tile_k, void* stream, char* err, size_t errlen);
/* @batch_matmul (arg0, arg1, arg2) -- examples/bmm_2Dmesh/IR/00_from_helion_frontend.mlir:4 */
int loom_hip_ciface_batch_matmul(const loom_memref3_t* arg0, const loom_memref3_t* arg1,
                                 const loom_memref3_t* arg2, int64_t tile_b, int64_t tile_m,
                                 int64_t tile_n, int64_t tile_k, void* stream, char* err,
                                 size_t errlen);
int loom_hip_ciface_batch_matmul_f16(const loom_memref3_t* arg0, const loom_memref3_t* arg1,
                                     const loom_memref3_t* arg2, int64_t tile_b, int64_t tile_m,
                                     int64_t tile_n, int64_t tile_k, void* stream, char* err,
                                     size_t errlen);
/* @split_k_matmul_gather (a, b, out) -- examples/split_k_mm_gather/IR/00_from_helion_frontend.mlir:2;
 * the gathered partial stack stays a workspace as for the pointer form. */
int loom_hip_ciface_split_k_matmul_gather(const loom_memref2_t* a, const loom_memref2_t* b,
                                          const loom_memref2_t* out, void* partials,
                                          size_t partials_bytes, int64_t tile_m, int64_t tile_n,
                                          int64_t tile_k, void* stream, char* err, size_t errlen);
int loom_hip_ciface_split_k_matmul_gather_f16(const loom_memref2_t* a, const loom_memref2_t* b,
                                              const loom_memref2_t* out, void* partials,
                                              size_t partials_bytes, int64_t tile_m,
                                              int64_t tile_n, int64_t tile_k, void* stream,
                                              char* err, size_t errlen);
/* @attention (k, v, q, out) -- examples/flashattn/IR/00_from_helion_frontend.mlir:4 */
int loom_hip_ciface_attention(const loom_memref3_t* k, const loom_memref3_t* v,
                              const loom_memref3_t* q, const loom_memref3_t* out, float scale,
                              int causal, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                              void* stream, char* err, size_t errlen);
int loom_hip_ciface_attention_f16(const loom_memref3_t* k, const loom_memref3_t* v,
                                  const loom_memref3_t* q, const loom_memref3_t* out, float scale,
                                  int causal, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                                  void* stream, char* err, size_t errlen);
/* @flash_decode (k, v, q, out) -- examples/mqa_decode/IR/00_from_helion_frontend.mlir:6 */
int loom_hip_ciface_flash_decode(const loom_memref3_t* k, const loom_memref3_t* v,
                                 const loom_memref3_t* q, const loom_memref3_t* out,
                                 void* workspace, size_t workspace_bytes, float scale,
                                 int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                 char* err, size_t errlen);
int loom_hip_ciface_flash_decode_f16(const loom_memref3_t* k, const loom_memref3_t* v,
                                     const loom_memref3_t* q, const loom_memref3_t* out,
                                     void* workspace, size_t workspace_bytes, float scale,
                                     int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                     char* err, size_t errlen);
/* @helion_mamba2_chunk_scan_kernel (cb, x, dt, dA_cumsum, C, D, prev_states_T, out) --
 * examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4 */
int loom_hip_ciface_helion_mamba2_chunk_scan_kernel(
    const loom_memref5_t* cb, const loom_memref4_t* x, const loom_memref4_t* dt,
    const loom_memref4_t* dA_cumsum, const loom_memref4_t* C, const loom_memref1_t* D,
    const loom_memref5_t* prev_states_T, const loom_memref4_t* out, int64_t tile_b,
    int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
    char* err, size_t errlen);
int loom_hip_ciface_helion_mamba2_chunk_scan_kernel_f16(
    const loom_memref5_t* cb, const loom_memref4_t* x, const loom_memref4_t* dt,
    const loom_memref4_t* dA_cumsum, const loom_memref4_t* C, const loom_memref1_t* D,
    const loom_memref5_t* prev_states_T, const loom_memref4_t* out, int64_t tile_b,
    int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
    char* err, size_t errlen);

/* loom_hip_dispatch over descriptors: `descs` points to the function's
 * memref descriptors in IR order, each of the rank its argument has
 * (loom_memref<R>_t); extents come from them.  Otherwise as
 * loom_hip_dispatch (the workspace carries split-K's partials or decode's
 * gathered splits). */
int loom_hip_dispatch_memref(const char* variant, const void* const* descs, int ndescs,
                             float scale, int causal, void* workspace, size_t workspace_bytes,
                             void* stream, char* err, size_t errlen);
int loom_hip_dispatch_memref_f16(const char* variant, const void* const* descs, int ndescs,
                                 float scale, int causal, void* workspace, size_t workspace_bytes,
                                 void* stream, char* err, size_t errlen);
/* Validates a descriptor call of loom_hip_dispatch_memref (f16 != 0: the
 * _f16 form) exactly as it would run -- descriptors, layouts, shapes, tiles,
 * scale -- and launches nothing (no device is needed). */
int loom_hip_check_memref(const char* variant, const void* const* descs, int ndescs, int f16,
                          float scale, char* err, size_t errlen);

/* ---- materialization contract and by-name dispatch ---------------------- */

/* Variant names the materialization pipeline emits for `funcs` under the
 * solver's block-size JSON, written to out[0..outlen) one per line in
 * emission order.  Follows run_materialization's input contract
 * (lib/pipeline/src/loom_materialization_pipeline.cpp:81-192): the root is an
 * object mapping a function name to a binding object {"sym": int}, a
 * non-empty array of binding objects, or null (UNSAT: no variant);
 * "__loom_candidate_order__" is an array of names that orders the functions
 * (unranked ones last); "ALL" binds every function without an entry of its
 * own and replaces the candidate order (:251-270).  An empty string selects
 * the placeholder solver (lib/passes/loom-opt/src/materialize.cpp:56-65) over
 * each example function's symbols.  Names are <func> + "__<sym><value>" in
 * sorted symbol order, "__combo<i>" added on a clash (materialize.cpp:39-53,
 * 253-262).  Rejections carry the reference's messages. */
int loom_hip_materialize_variants(const char* block_sizes_json, const char* const* funcs,
                                  int nfuncs, char* out, size_t outlen, char* err,
                                  size_t errlen);

/* Splits a materialized variant name into its function name (the text
 * before the first "__") and the tile_* values its suffix binds
 * (tiles[LOOM_HIP_TILE_*], -1 where unbound).  Other "__" tokens (mapping
 * variants such as "__d0i0_d1i0", "__combo<i>") are skipped.  Inverse of the
 * naming in materialize.cpp:39-53. */
int loom_hip_parse_variant(const char* variant, char* func, size_t funclen, int64_t* tiles,
                           char* err, size_t errlen);

/* Launches the kernel a materialized variant names: the step a gfx950
 * backend performs where the reference hands materialized IR to its TT
 * lowering (lib/pipeline/src/loom_materialization_pipeline.cpp:307-313).
 * `tensors` are the function's memref arguments in IR order; `dims` its
 * extents in the order of the matching entry point above:
 *   matmul (3 tensors) M,N,K | batch_matmul (3) B,M,N,K |
 *   split_k_matmul_gather (3) M,N,K (workspace = partials) |
 *   attention (4) BH,Sq,Skv,D (scale, causal used) |
 *   flash_decode (4) B,H,D,S (scale used; workspace as for that call) |
 *   helion_mamba2_chunk_scan_kernel (8) batch,nchunks,nheads,ngroups,
 *   chunk_size,headdim,dstate.
 * Every tile symbol the entry point takes must be bound by the name.
 * Unknown functions return LOOM_HIP_EUNSUP. */
int loom_hip_dispatch(const char* variant, void* const* tensors, int ntensors,
                      const int64_t* dims, int ndims, float scale, int causal, void* workspace,
                      size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* Bytes of the workspace loom_hip_dispatch needs for `variant` at `dims`
 * (the extents loom_hip_dispatch takes): split-K's fp32 partials (as
 * loom_hip_split_k_workspace_bytes at the name's tile_k), decode's
 * (lse_s, o_s) (as loom_hip_flash_decode_workspace_bytes at its tile_s), 0
 * for the other functions.  The generic form of the two per-function
 * queries, for a caller that holds only the materialized name. */
int loom_hip_workspace_bytes(const char* variant, const int64_t* dims, int ndims,
                             size_t* bytes, char* err, size_t errlen);

/* loom_hip_dispatch for variants whose 16-bit tensors are f16 (the
 * reference's own element type): launches the *_f16 entry points. */
int loom_hip_dispatch_f16(const char* variant, void* const* tensors, int ntensors,
                          const int64_t* dims, int ndims, float scale, int causal,
                          void* workspace, size_t workspace_bytes, void* stream, char* err,
                          size_t errlen);

/* Validates a materialized variant against its extents exactly as
 * loom_hip_dispatch would -- same checks, same codes and messages -- and
 * launches nothing (no device is needed).  `dims` as for loom_hip_dispatch. */
int loom_hip_check_variant(const char* variant, const int64_t* dims, int ndims, char* err,
                           size_t errlen);

/* ---- gfx950 block-size constraints for the external solver ---------------
 * The reference hands its solver one constraint scope per variant
 * (examples/mm/constraint_space/staged_etg_dump.json; built in
 * lib/passes/lcs/src/staged_etg_builder.cpp:1465-1478 and
 * hard_constraint_pipeline.cpp:162-213) with Tenstorrent rules: inner tile
 * dims aligned to 32 (hw_alignment.cpp:16) and an L1 budget of 1499136 bytes.
 * loom_hip_constraint_scope writes the same JSON object for gfx950 --
 * {"variant_name", "constraint_scope": {"metadata": {"datatype", "booleans",
 * "iter_num", "L1_footprint" (LDS bytes here), "symbols": {sym: {"type",
 * "natural_ub", "alignment"}}}, "hard_constraints": [...]}} in the grammar of
 * lib/passes/lcs/inc/expr.h and constraint_expr.h -- whose hard constraints
 * accept exactly the bindings this library builds for those extents (the
 * workgroup tiles of each kernel, LDS <= 160 KiB).  `dims` as for
 * loom_hip_dispatch; a shape no kernel supports returns LOOM_HIP_EUNSUP. */
int loom_hip_constraint_scope(const char* func, const int64_t* dims, int ndims, char* out,
                              size_t outlen, char* err, size_t errlen);

/* The MI355X machine model the constraint scopes are written against, as
 * JSON: LDS bytes per workgroup (the footprint constraint's capacity), wave
 * size, SIMDs, MFMA shapes, the workgroup tiles each kernel builds and the
 * published peaks; with device >= 0 also what that device reports (CU count,
 * LDS per CU and per workgroup, L2, memory, clock), code 3 if it cannot be
 * queried.  The counterpart of the reference's --hw_spec machine description
 * (R/run_pipeline.sh:62,93, a 2-D mesh file in an external grammar) for
 * this target. */
int loom_hip_hw_spec(int device, char* out, size_t outlen, char* err, size_t errlen);

/* The binding this library runs fastest for those extents on MI355X (one
 * JSON object {"tile_m": 256, ...} over the function's symbols; a legal
 * point of loom_hip_constraint_scope), usable as a block_sizes_json entry. */
int loom_hip_preferred_block_sizes(const char* func, const int64_t* dims, int ndims, char* out,
                                   size_t outlen, char* err, size_t errlen);

/* ---- on-box ceilings ---------------------------------------------------
 * Measurement kernels with no counterpart in the reference: what one part
 * sustains, next to the published peaks the roofline fractions use.
 * loom_hip_peak_hbm_read streams `bytes` of `buf` (16-byte aligned) once;
 * its rate is bytes / kernel time.  loom_hip_peak_mfma_bf16 runs `iters`
 * rounds of independent bf16 MFMA chains on every CU and stores the FLOP it
 * performs in *flop; its rate is *flop / kernel time.  `sink` is a device
 * word the kernels may write (so their work cannot be optimised away). */
int loom_hip_peak_hbm_read(const void* buf, size_t bytes, void* sink, void* stream, char* err,
                           size_t errlen);
int loom_hip_peak_mfma_bf16(int64_t iters, void* sink, double* flop, void* stream, char* err,
                            size_t errlen);

/* ---- synthetic inputs --------------------------------------------------
 * No counterpart in the reference: the measurement's seeded inputs.  Writes
 * n elements (bf16 bits if bf16 != 0, else fp32) of stream `seed` of a
 * counter-based generator: dist 0 uniform in [a, b), dist 1 normal with
 * mean a and standard deviation b.  Element i depends on (seed, i) only and
 * is bit-identical to the CPU oracle's loom_oracle_synth. */
int loom_hip_synth(void* out, int64_t n, uint64_t seed, int dist, float a, float b, int bf16,
                   void* stream, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* LOOM_HIP_H */
