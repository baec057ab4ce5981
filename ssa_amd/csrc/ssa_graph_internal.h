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
