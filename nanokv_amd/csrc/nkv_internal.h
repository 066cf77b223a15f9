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
    int r, group, scale_dtype, id_bytes, num_centers, _pad;
    const uint16_t* w;        // bf16 row d of head i: w + i*w_hs + d*r
    int64_t w_hs;
    const uint16_t* centers;  // bf16 value (b, id, i, d): centers[b*c_bs + id*c_rs + i*c_hs + d];
    int64_t c_bs, c_rs, c_hs;  // null = no center add
    const float* bias;        // (i, d): bias[i*bias_hs + d], applied as bf16; null = none
    int64_t bias_hs;
};

// One key-chunk attention launch: every launch head i attends queries
// q[b, :, i, :dk] to the history keys rows[0 .. n_rows) (decoded with the
// codec tables, K to width dk, V to width 128) and the current keys
// k_cur/v_cur[b, 0 .. Nc, i]; out[b, :, i, :128] bf16, lse[b, i, :] natural
// log (or null).
struct ChunkLaunchDesc {
    int B, H, dk;
    int64_t Q, N, n_rows, Nc;
    const int32_t* rows;
    float softmax_scale;
    const uint16_t* q;
    int64_t q_sb, q_st, q_sh;
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
};

// The decoder view of an nkv_codec for head dim D: head h reads decoder rows
// h*D .., center columns h*D .. and mean h*D ...
ChunkCodec chunk_codec_from(const nkv_codec& c, int D, int HD);

// Key-chunk schedule (nkv_chunk.hip).
int chunk_check(const nkv_attend_args* a);
size_t chunk_workspace_bytes(const nkv_attend_args* a);
int chunk_attend_launch(hipStream_t s, const nkv_attend_args* a, void* workspace,
                        size_t workspace_bytes);
size_t chunk_launch_workspace(const ChunkLaunchDesc& d);
int chunk_launch(hipStream_t s, const ChunkLaunchDesc& d, void* workspace, size_t workspace_bytes);

}  // namespace nkv
