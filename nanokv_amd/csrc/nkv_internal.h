// nkv_internal.h -- types and entry points shared between the translation
// units of libnanokv_hip.so (not part of the C ABI).
#pragma once

#include "nkv_common.h"
#include "nkv_camera.h"
#include "nkv_rope.h"

namespace nkv {

// One K or V codec as a key-chunk launch reads it: the history's packed
// codes, scales and center ids (shared by every head), and the decode tables
// of each launch head i (decoder or reader rows, center columns, bias).
struct ChunkCodec {
    const uint8_t* packed;    // [B, N, r/2]
    const uint16_t* scales;   // [B, N, r/group]
    const void* ids;          // [B, N] of id_bytes, or null
    int r, group, scale_dtype, id_bytes, num_centers;
    int has_centers;          // 1: add each row's center (flat table or the segments' tables)
    const uint16_t* w;        // bf16 row d of head i: w + i*w_hs + d*r
    int64_t w_hs;
    const uint16_t* centers;  // bf16 value (b, id, i, d): centers[b*c_bs + id*c_rs + i*c_hs + d]
    int64_t c_bs, c_rs, c_hs;
    const float* bias;        // (i, d): bias[i*bias_hs + d], applied as bf16; null = none
    int64_t bias_hs;
    // Head of the center table and bias of launch head i: c_heads[i] clamped
    // to [0, c_heads_n) (null: i).  Lets a launch over a subset of a layer's
    // heads read the layer's own tables; honoured by the resident-decoder
    // tile kernel only (the staged schedule's decode GEMM).
    const int32_t* c_heads;
    int c_heads_n;
    // Segment table in device memory (null: the flat arrays above).  Row n of
    // batch item b lives in segment s = seg_find(n) at local row n - row_start.
    // seg_flat == 0: its center is (b, id) of the segment's own table
    // (segment centers + b*centers_batch_stride + id*c_rs + i*c_hs + d);
    // seg_flat == 1: row center_base + id of the one table `centers` above.
    const nkv_segment* seg;
    int n_seg;
    int seg_flat;
};

// Segment holding codec row `row` of a table in row order, contiguous from
// row 0 (binary search; rows outside the table give its first or last).
__device__ __forceinline__ int seg_find(const nkv_segment* seg, int n, int64_t row) {
    const NKV_GLOBAL nkv_segment* sg = (const NKV_GLOBAL nkv_segment*)seg;
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sg[mid].row_start <= row) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Segment `i` of a device segment table, read as global memory.
__device__ __forceinline__ const NKV_GLOBAL nkv_segment& seg_at(const nkv_segment* seg, int i) {
    return ((const NKV_GLOBAL nkv_segment*)seg)[i];
}

// Packed-code and scale rows of codec row `row` of batch item b (N rows per
// batch item in the flat layout).
__device__ __forceinline__ void codec_row_ptrs(const ChunkCodec& c, int b, int64_t N, int64_t row,
                                               const uint8_t*& prow, const uint16_t*& srow) {
    const int NG = c.r / c.group;
    if (c.seg) {
        const NKV_GLOBAL nkv_segment& s = seg_at(c.seg, seg_find(c.seg, c.n_seg, row));
        const int64_t local = min(max(row - s.row_start, (int64_t)0), s.rows - 1);
        const int64_t tok = (int64_t)b * s.rows + local;
        prow = s.packed + tok * (c.r / 2);
        srow = s.scales + tok * NG;
    } else {
        const int64_t tok = (int64_t)b * N + row;
        prow = c.packed + tok * (c.r / 2);
        srow = c.scales + tok * NG;
    }
}

// Center row (bf16, the launch head's columns) of codec row `row` of batch
// item b; ids outside a table are clamped so that a corrupt payload cannot
// read out of bounds.  Only for codecs with has_centers.
__device__ __forceinline__ const uint16_t* center_row(const ChunkCodec& c, int b, int h, int64_t N,
                                                      int64_t row) {
    if (c.seg) {
        const NKV_GLOBAL nkv_segment& s = seg_at(c.seg, seg_find(c.seg, c.n_seg, row));
        const int64_t local = min(max(row - s.row_start, (int64_t)0), s.rows - 1);
        int id = read_id(s.ids, s.id_bytes, (int64_t)b * s.rows + local);
        id = min(max(id, 0), s.num_centers - 1);
        if (c.seg_flat)
            return c.centers + (int64_t)b * c.c_bs + (s.center_base + id) * c.c_rs + (int64_t)h * c.c_hs;
        return s.centers + (int64_t)b * s.centers_batch_stride + (int64_t)id * c.c_rs +
               (int64_t)h * c.c_hs;
    }
    int id = read_id(c.ids, c.id_bytes, (int64_t)b * N + row);
    id = min(max(id, 0), c.num_centers - 1);
    return c.centers + (int64_t)b * c.c_bs + (int64_t)id * c.c_rs + (int64_t)h * c.c_hs;
}

// One key-chunk attention launch: every launch head i attends queries
// q[b, :, i, :dk] to the history keys rows[0 .. n_rows) (decoded with the
// codec tables, K to width dk, V to width 128) and the current keys
// k_cur/v_cur[b, 0 .. Nc, i]; out[b, :, i, :128] bf16, lse[b, i, :] natural
// log (or null).
// Partitions of one multi-partition staged launch (a NanoKV-Fast call's
// native partition and reader groups).
constexpr int NKV_MAX_PARTS = 4;

struct ChunkLaunchDesc {
    int B, H, dk;
    int64_t Q, N, n_rows, Nc;
    const int32_t* rows;
    float softmax_scale;
    const uint16_t* q;
    int64_t q_sb, q_st, q_sh;
    // query head of launch head i: q_heads[i] clamped to [0, q_heads_n)
    // (null: i); staged schedule only
    const int32_t* q_heads;
    int q_heads_n;
    const uint16_t* k_cur;
    int64_t k_sb, k_st, k_sh;
    const uint16_t* v_cur;
    int64_t v_sb, v_st, v_sh;
    ChunkCodec key, value;
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    void* ev_begin;  // optional hipEvent_t recorded around the attention kernel
    void* ev_end;
    RopeDev rope;    // RoPE of the history keys at their codec rows (cs_t null: none)
    CameraDev cam;   // camera P^-1 of the history keys and values (mats null: none)
    // visibility of the current keys: bit k % 32 of cur_mask[g * mask_words +
    // k / 32] for the queries of group g = q_group[t] (null: all visible)
    const uint32_t* cur_mask;
    const int32_t* q_group;
    int n_groups, mask_words;
};

// The decoder view of an nkv_codec for head dim D: head h reads decoder rows
// h*D .., center columns h*D .. and mean h*D ...
ChunkCodec chunk_codec_from(const nkv_codec& c, int D, int HD);

// Whether rows of a [B, T, H, D] bf16 tensor can be read and written as
// 16-byte pieces (the kernels' query, output and current-key accesses).
inline bool rows16(const void* p, int64_t sb, int64_t st, int64_t sh) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && sb % 8 == 0 && st % 8 == 0 && sh % 8 == 0;
}

// Host check of a codec's segment table against its N rows (NKV_OK when the
// codec has no segments).
int check_segments(const nkv_codec& c, int64_t N);

// Key-chunk schedule (nkv_chunk.hip).
int chunk_check(const nkv_attend_args* a);
size_t chunk_workspace_bytes(const nkv_attend_args* a);
int chunk_attend_launch(hipStream_t s, const nkv_attend_args* a, void* workspace,
                        size_t workspace_bytes);
size_t chunk_launch_workspace(const ChunkLaunchDesc& d);
int chunk_launch(hipStream_t s, const ChunkLaunchDesc& d, void* workspace, size_t workspace_bytes);

// Partitions d[0 .. n) of one attention call through the staged schedule in
// one decode, one flash and one combine launch (the decode in two when the
// codecs' ranks differ).  Partition 0 (128 wide) covers every head of the
// layer; the combine writes the merged output and LSE to its out / lse.
// Partition i >= 1 covers heads heads[i][0 .. d[i].H) of the layer (the first
// partition listing a head is merged into it; heads outside the layer are
// never merged), its output shifted by shift[b*sh_sb + h*sh_sh + e] (null:
// none) before the merge; with ocam.mats set, the merged output is then
// multiplied by P of its query row (FULL layout).  Supported: every
// partition staged by the decode GEMM (ranks <= 384, the camera only in the
// FULL layout, the same codec ranks, B and Q), current keys in partition 0
// only.
bool staged_multi_supported(const ChunkLaunchDesc* d, int n);
size_t staged_multi_workspace(const ChunkLaunchDesc* d, int n);
int staged_multi_launch(hipStream_t s, const ChunkLaunchDesc* d, int n, const int32_t* const* heads,
                        const float* shift, int64_t sh_sb, int64_t sh_sh, void* workspace,
                        size_t workspace_bytes, const CameraDev& ocam);

}  // namespace nkv
