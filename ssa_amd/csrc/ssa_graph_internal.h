// ssa_graph_internal.h -- launchers shared between the graph-build sources.
#pragma once

#include "ssa_common.h"
#include "../../include/ssa_amd.h"

// LDS a workgroup may use on gfx950 (160 KiB), minus room for static shared data
#define SSA_LDS_BYTES (160 * 1024 - 512)

int ssa_sort_supported(int n);
int64_t ssa_sort_tmp_bytes(int rows, int n);
// the segment counter inside the sort's scratch `tmp`: it must be 0 when the
// sort starts (counter_clear: the sort clears it itself; else the caller has)
int32_t *ssa_sort_counter(uint16_t *tmp, int rows, int n);
// The bucket sort's top levels as a caller launches them itself (rows of at
// most 32768 keys: 16-bit positions, the row in LDS): sort_top_row's
// arguments and the dynamic LDS it needs; the caller then runs the segment
// pass (sort_seg_blocks<uint16_t>) over ssa_sort_seg_blocks() workgroups.
struct SortTopArgs {
    const uint16_t *ids;
    int rows, n, NB;
    int32_t *perm, *bstart, *bsize;
    uint32_t *gkv;
    int4 *segs;
    int *segcount;
    unsigned char *glb;
    int tl_in_lds, cap, lds;
};
int ssa_sort_top_setup(const uint16_t *ids, int rows, int n, int P, int32_t *perm,
                       int32_t *bstart, int32_t *bsize, uint16_t *tmp, SortTopArgs *a);
// workgroups of the segment launch (SEG_WAVES waves each) for rows x n keys
int ssa_sort_seg_blocks(int rows, int n);
int ssa_launch_bucket_sort(const uint16_t *ids, int rows, int n, int P, int32_t *perm,
                           int32_t *bstart, int32_t *bsize, uint16_t *tmp, hipStream_t st,
                           bool counter_clear = true);

// The graph build with its workspace held to ws_cap bytes (query heads in
// chunks that fit): the workspace size it needs (or a negative SSA_E_* code,
// SSA_E_WORKSPACE when one head per chunk does not fit), and the build over a
// workspace of ws_cap bytes.
int64_t ssa_graph_workspace_bytes_capped(const ssa_graph_args *a, int64_t ws_cap);
int ssa_build_graph_capped(const ssa_graph_args *a, void *workspace, int64_t ws_cap,
                           void *stream);

// ---------------------------------------------------------------------------
// The projections with the hash in their epilogue (ssa_proj.hip).
#define SSA_PROJ_PLAIN 0     // Y = X W^T only
#define SSA_PROJ_KEYS 1      // + key bucket ids and the 16-row maxima of |k|^2
#define SSA_PROJ_QUERIES 2   // + query bucket / probe ids, code scales, aux scores

struct ProjP {
    const void *x; int64_t ldx;        // (rows, K) bf16, row stride ldx elements
    const void *w; int64_t ldw;        // (cols, K) bf16
    void *y; int64_t ldy;              // (rows, cols) bf16, written
    int rows, cols, K;
    int mode;
    int L;                             // positions per batch: rows = B * L
    int Lk;                            // QUERIES: key positions per batch (rows of k)
    int d;                             // head dim (epilogue)
    int heads;                         // KEYS: kv heads hashed (columns [0, heads * d))
    const uint16_t *psplit;            // hyperplanes as 3 bf16 terms (ssa_launch_plane_split)
    int R, P, Tp, NS;
    uint16_t *ids;                     // KEYS: (B*Hkv*R, L); QUERIES: (B*Hq*L, R, NS)
    uint32_t *kpart;                   // KEYS: max |k|^2 of each 16 rows of a kv head
    int32_t *zero1;                    // cleared by block 0 (a later kernel's counter)
    // QUERIES: the keys (the kv projection's output) and the aux rows
    const void *k; int64_t ksb, ksh, ksn;
    const int64_t *glob;
    int G, NA, causal, Hq, Hkv, rep;
    const uint32_t *knorm;             // max |k|^2 per (batch, kv head)
    float *aux;                        // (B*Hq*L, NA)
};

// whether the hash epilogue takes these sizes (rows = B * L, cols = heads * d,
// K = d_model, np = R * P hyperplanes)
bool ssa_project_supported(int rows, int cols, int K, int d, int np);
int64_t ssa_plane_split_bytes(int np, int d);
int ssa_launch_plane_split(const float *planes, int R, int maxP, int P, int d, uint16_t *out,
                           hipStream_t st);
int ssa_launch_project(const ProjP &p, hipStream_t st);
