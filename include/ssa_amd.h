/*
 * ssa_amd.h -- C ABI of the MI355X (gfx950) SparseAttention forward hot path.
 *
 * One shared library, libssa_amd.so, exports the functions below.  Every entry
 * point takes plain pointers, element strides and sizes; nothing here knows
 * about torch.  Device pointers are HIP device addresses; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  All work is
 * enqueued on `stream`; no entry point synchronises the host, allocates device
 * memory or frees caller memory.  Callers own every buffer (inputs, outputs,
 * workspace).  Every function returns 0 on success and a negative SSA_E_*
 * code otherwise; ssa_last_error() returns a message for the calling thread's
 * last failure.
 *
 * The entry points replace the reference's Python functions (daedalus/SSA,
 * sparse_attention.py) cited on each declaration.
 */
#ifndef SSA_AMD_H
#define SSA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of q / k / v / out */
#define SSA_F32  0
#define SSA_BF16 1
#define SSA_F16  2

/* status codes */
#define SSA_OK          0
#define SSA_E_ARG      -1   /* invalid argument (shape, stride, dtype)        */
#define SSA_E_UNSUP    -2   /* unsupported size (head dim, bucket bits, ...)  */
#define SSA_E_WORKSPACE -3  /* workspace too small                           */
#define SSA_E_HIP      -4   /* a HIP runtime call failed                      */

/* A (B, Hx, L, d) tensor view with the last dimension contiguous.  Strides are
 * in elements.  Head h of a query tensor reads kv head h / (Hq / Hkv). */
typedef struct {
    const void *ptr;
    int32_t dtype;           /* SSA_F32 / SSA_BF16 / SSA_F16 */
    int64_t sb, sh, sn;      /* strides of B, head, position */
} ssa_tensor4;

/* ---------------------------------------------------------------------------
 * Neighbor-graph build.
 *
 * mode SSA_GRAPH_FULL replaces SparseAttention.build_graph
 *   (sparse_attention.py:1325-1390: window + global + LSH + self, merged by
 *   merge_neighbors :966-1089).  Outputs neighbors (B,Hq,N,k_out) int64 and
 *   valid (B,Hq,N,k_out) uint8 with k_out = ssa_graph_out_width().
 * mode SSA_GRAPH_LSH replaces LSHGraphBuilder.forward
 *   (sparse_attention.py:814-959).  Outputs lsh_idx (B,Hq,N,kk) int64,
 *   kk = min(top_k, R*(1+min(T,P))*C), ordered by descending score; slots
 *   without a candidate hold glob[t] (t < G) or 0, as the reference does.
 *
 * k may be the un-expanded (B, Hkv, M, d) tensor: query head h uses kv head
 * h / (Hq / Hkv).  Passing an already expanded k (Hkv = Hq) is also valid.
 * --------------------------------------------------------------------------- */
#define SSA_GRAPH_FULL 0
#define SSA_GRAPH_LSH  1

typedef struct {
    int32_t mode;            /* SSA_GRAPH_FULL / SSA_GRAPH_LSH                       */
    int32_t B, Hq, Hkv;      /* batch, query heads, kv heads (Hq % Hkv == 0)         */
    int32_t N, M, d;         /* query length, key length, head dim                   */
    ssa_tensor4 q;           /* (B, Hq, N, d)                                        */
    ssa_tensor4 k;           /* (B, Hkv, M, d)                                       */
    const float *rand_proj;  /* (R, max_p, d) fp32 hyperplanes, contiguous           */
    int32_t R, max_p;        /* rounds, planes registered per round                  */
    int32_t P;               /* effective planes this call (1..12)                   */
    int32_t T;               /* requested probes (clamped to P internally)            */
    int32_t C;               /* candidates per bucket list (lsh_candidates)          */
    int32_t top_k;           /* LSH top-k (lsh_k)                                    */
    int32_t window;          /* window half width w (FULL, self-attention only)      */
    int32_t causal;          /* future candidates -> self, causal window             */
    int32_t is_cross;        /* cross-attention: no window, no self slot             */
    int32_t total_k;         /* num_neighbors K (FULL)                               */
    const int64_t *glob;     /* (G,) global key ids, already clamped to [0, M-1]     */
    int32_t G;
    /* Optional injected fp32 projections (parity testing):                          */
    const float *q_proj;     /* (B*Hq, R, N, P) or NULL                              */
    const float *k_proj;     /* (B*Hkv, R, M, P) or NULL                             */
    /* outputs */
    int64_t *out_idx;        /* FULL: neighbors (B,Hq,N,k_out); LSH: (B,Hq,N,kk)     */
    uint8_t *out_valid;      /* FULL: (B,Hq,N,k_out); LSH: unused (may be NULL)      */
    int32_t *out_ties;       /* optional single counter (caller zeroes it): queries   */
                             /* whose kk-th LSH score is tied; their selection is     */
                             /* replayed with the reference's top-k tie order         */
    /* FULL mode, optional (no counterpart in the reference): the same graph as   */
    /* (B,Hq,N,k_out) int32 ids with -1 in the invalid slots, for callers that    */
    /* only hand the graph to ssa_sparse_gather_attention; when set, out_idx and */
    /* out_valid are not written and may be NULL.                                */
    int32_t *out_idx32;
} ssa_graph_args;

/* Output width of the FULL graph: self-attention 1 + min(K-1, 2w+1+G+kk),
 * cross-attention min(K, G+kk) (sparse_attention.py:1062-1072). */
int64_t ssa_graph_out_width(const ssa_graph_args *a);

/* Bytes of device workspace ssa_build_graph needs for these arguments. */
int64_t ssa_graph_workspace_bytes(const ssa_graph_args *a);

/* Replaces SparseAttention.build_graph (:1325-1390) and, in SSA_GRAPH_LSH
 * mode, LSHGraphBuilder.forward (:814-959). */
int ssa_build_graph(const ssa_graph_args *a, void *workspace, int64_t workspace_bytes,
                    void *stream);

/* ssa_build_graph without any device allocation (no counterpart in the
 * reference): for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The same
 * arguments, outputs and results as ssa_build_graph, but the workspace is a
 * fixed array of SSA_NOALLOC_SCRATCH_BYTES in device memory that the library
 * holds on every GPU it runs on until the process ends.  Query heads are built
 * in chunks small enough for it; a problem that needs more than the array with
 * one query head per chunk fails with SSA_E_WORKSPACE before any launch.  The
 * caller still allocates the outputs.  `stream` must belong to the current
 * device.  All calls on one GPU share its array: calls that overlap on one GPU
 * (other streams, other host threads) race and must not be issued. */
#define SSA_NOALLOC_SCRATCH_BYTES (64 << 20)
int ssa_build_graph_noalloc(const ssa_graph_args *a, void *stream);

/* ---------------------------------------------------------------------------
 * Projections and graph build in one call (bf16 models).
 *
 * Replaces the q / k / v projections of SparseAttention.forward
 * (sparse_attention.py:1484-1486, Wq(x), Wk(src), Wv(src)) followed by
 * build_graph (:1325-1390).  The projections run on the library's own
 * matrix-core GEMM, whose epilogue computes from each output tile what the
 * build would otherwise read q and k again for: the bucket and probe ids of
 * every row (_hash_proj / _hash / _probe_ids, :559-646, as :775-779 call
 * them), the keys' norms and the query-side scores the candidate lists do
 * not carry.  Same outputs as ssa_build_graph on the q and k it writes.
 *   x       (B, N, d_model) bf16, rows d_model elements apart
 *   src     (B, M, d_model) bf16 (x itself for self-attention)
 *   wq      (Hq*d, d_model) bf16 row-major (Wq.weight)
 *   wkv     (2*Hkv*d, d_model) bf16 row-major: Wk.weight's rows, then Wv.weight's
 *   q_out   (B, N, Hq*d) bf16, written (x Wq^T)
 *   kv_out  (B, M, 2*Hkv*d) bf16, written (src [Wk; Wv]^T: k, then v, per row)
 *   graph   the build's arguments; graph.q and graph.k must be the
 *           (B, Hq, N, d) and (B, Hkv, M, d) views of q_out and kv_out,
 *           graph.q_proj / k_proj NULL.
 * All pointers 16-byte aligned.  ssa_project_graph_supported() returns 1 when
 * these sizes take this path: bf16, d 32 / 64 / 128, N and M multiples of 16,
 * d_model a multiple of 64, Hq*d and 2*Hkv*d multiples of 256, R*P at most
 * 48 (d 128), 64 (d 64, 32) hyperplanes; else 0 (use the projections of the
 * caller's choice and ssa_build_graph).
 * --------------------------------------------------------------------------- */
typedef struct {
    const void *x, *src, *wq, *wkv;
    void *q_out, *kv_out;
    int32_t d_model;
    ssa_graph_args graph;
} ssa_project_graph_args;

int ssa_project_graph_supported(const ssa_project_graph_args *a);
int64_t ssa_project_graph_workspace_bytes(const ssa_project_graph_args *a);
int ssa_project_build_graph(const ssa_project_graph_args *a, void *workspace,
                            int64_t workspace_bytes, void *stream);

/* The bf16 projection GEMM alone (no counterpart in the reference; exposed to
 * test it): y (rows, cols) = x (rows, K) w (cols, K)^T, fp32 accumulation,
 * rounded once to bf16.  cols a multiple of 256, K of 64; row strides in
 * elements, multiples of 8; pointers 16-byte aligned. */
int ssa_project_gemm(const void *x, int64_t ldx, const void *w, int64_t ldw, void *y,
                     int64_t ldy, int32_t rows, int32_t cols, int32_t K, void *stream);

/* ---------------------------------------------------------------------------
 * Bucket permutation: for each of `rows` rows of `n` bucket ids (uint16, values
 * < 2^P), the permutation torch.sort(ids, dim=-1) returns on the CPU (an
 * unstable introsort; sparse_attention.py:781), plus bucket start / size
 * tables (:785-792).  Bucket starts of empty buckets hold the next bucket's
 * start.  Exposed for testing the sort stage on its own.
 * --------------------------------------------------------------------------- */
int64_t ssa_bucket_sort_workspace_bytes(int32_t rows, int32_t n);
int ssa_bucket_sort(const uint16_t *ids, int32_t rows, int32_t n, int32_t P,
                    int32_t *perm, int32_t *bstart, int32_t *bsize,
                    void *workspace, int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Merge of arbitrary window / global / LSH index lists.
 * Replaces merge_neighbors (sparse_attention.py:966-1089).
 *   win (N, Kw) int64 contiguous (Kw may be 0), glob (G,), lsh (BH, N, Kl)
 *   contiguous.  has_self: self-attention (slot 0 = n, n removed from pool).
 *   Outputs (BH, N, k_out) int64 + uint8 valid, k_out = has_self ?
 *   1 + min(K-1, Kw+G+Kl) : min(K, Kw+G+Kl).  workspace: 16 bytes.
 * --------------------------------------------------------------------------- */
int ssa_merge_neighbors(const int64_t *win, int32_t Kw, const int64_t *glob, int32_t G,
                        const int64_t *lsh, int32_t Kl, int32_t BH, int32_t N,
                        int32_t has_self, int32_t total_k, int64_t *out, uint8_t *valid,
                        void *workspace, void *stream);

/* ---------------------------------------------------------------------------
 * Gather attention.  Replaces sparse_gather_attention
 * (sparse_attention.py:1096-1199).
 *   q (B,Hq,N,d), k/v (B,Hkv,M,d) views; neighbors (B,Hq,N,K) int64 and
 *   valid (B,Hq,N,K) uint8 (or NULL = all valid), both contiguous.
 *   out: (B,Hq,N,d) in q's dtype written through the given strides.
 *   scores = fp32(q.k) * scale, masked to -inf where !valid, fp32 softmax;
 *   16-bit models round p to the value dtype before P.V unless fp32_weights;
 *   P.V accumulates in fp32 and rounds once.
 *   dropout_p > 0 applies inverted dropout to p with a counter-based hash of
 *   (seed, query row, slot).
 * --------------------------------------------------------------------------- */
typedef struct {
    int32_t B, Hq, Hkv, N, M, d, K;
    ssa_tensor4 q, k, v;
    const int64_t *neighbors;
    const uint8_t *valid;
    float scale;
    int32_t fp32_weights;
    float dropout_p;
    uint64_t seed;
    void *out;               /* dtype of q */
    int64_t out_sb, out_sh, out_sn;
    /* optional (no counterpart in the reference): the graph as int32 ids, a     */
    /* negative id marking an invalid slot (ssa_graph_args.out_idx32); when set, */
    /* neighbors and valid are not read.  Not accepted by the backward.          */
    const int32_t *neighbors32;
    /* optional (no counterpart in the reference): B*Hq*N int32, written with    */
    /* each query row's count of slots the graph marks invalid (valid false, or  */
    /* a negative id in neighbors32): the reference's padding statistic          */
    /* (sparse_attention.py:1500-1508) without a pass of its own over the graph. */
    /* An out-of-range id marked valid is skipped by the attention (as masked)   */
    /* but not counted.  Forward only.                                           */
    int32_t *row_invalid;
} ssa_apply_args;

int ssa_sparse_gather_attention(const ssa_apply_args *a, void *stream);

/* Backward of ssa_sparse_gather_attention (the graph is not differentiable,
 * sparse_attention.py:157-159): given dout (B,Hq,N,d) contiguous fp32 (the
 * upstream gradient), writes dq (B,Hq,N,d) fp32 and ACCUMULATES dk, dv
 * (B,Hkv,M,d) fp32 (the caller zeroes them).  Uses the same dropout seed. */
typedef struct {
    ssa_apply_args fwd;
    const float *dout;
    float *dq, *dk, *dv;
} ssa_apply_bwd_args;

int ssa_sparse_gather_attention_bwd(const ssa_apply_bwd_args *a, void *stream);

/* Deterministic backward (the reference's CPU autograd through
 * sparse_attention.py:1146-1199 is deterministic; ssa_sparse_gather_attention_bwd
 * adds dk / dv with fp32 atomics, whose order varies).  Same arguments and
 * results; each key row's terms are rounded to a fixed-point grid of that
 * row (the finest for which slot count x largest weight x largest |q| or
 * |dout| cannot overflow 64 bits) and summed as integers, so every run gives
 * the same bits.  Needs a 256-byte aligned workspace of
 * ssa_sparse_gather_attention_bwd_det_workspace_bytes (8 bytes per slot, 16
 * per key row element and 12 per key row); a key row whose bound is not
 * finite gets NaN.  SparseAttention takes it under
 * torch.use_deterministic_algorithms(True). */
int64_t ssa_sparse_gather_attention_bwd_det_workspace_bytes(const ssa_apply_bwd_args *a);
int ssa_sparse_gather_attention_bwd_det(const ssa_apply_bwd_args *a, void *workspace,
                                        int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Measurement helper (no counterpart in the reference): the L2-to-CU delivery
 * rate that bounds the gather attention, whose repeated K/V rows are served by
 * the L2 rather than HBM.  `blocks` workgroups of 256 threads each stream the
 * `bytes` of `buf` (a power of two, 32 KiB .. 2 GiB; small enough to stay in
 * the L2, larger than a CU's L1) `iters` times with 16-byte loads.  Bytes
 * delivered = blocks * bytes * iters.  `sink` holds `blocks` uint32 (written
 * only in a case the kernel never meets).
 * --------------------------------------------------------------------------- */
int ssa_measure_l2_read(const void *buf, int64_t bytes, int32_t blocks, int32_t iters,
                        uint32_t *sink, void *stream);

/* ---------------------------------------------------------------------------
 * Bounds-checked build (no counterpart in the reference): libssa_amd_checked.so
 * (`make -C ssa_amd/csrc checked`) is this library with the graph build's
 * data-dependent indices (key ids, sorted-list and bucket positions, tie rows,
 * output slots on the select, tie replay and merge paths) compared with the
 * length of what they index; an index outside is recorded and replaced by 0,
 * so no access leaves its buffer.  ssa_checked_oob synchronizes the device,
 * copies the record into record[4] (bit i of record[0]: site i saw an index
 * outside; record[1..3]: the last offender's site, index and length), clears
 * it and returns 1; in the product build it returns 0 and writes nothing.
 * --------------------------------------------------------------------------- */
int ssa_checked_oob(uint32_t *record);

/* Library identification and error text. */
const char *ssa_version(void);
const char *ssa_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* SSA_AMD_H */
