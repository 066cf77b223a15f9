// nkv_camera.h -- camera PRoPE transforms shared by the fused key-chunk kernel
// and nkv_camera_apply.
//
// prope_attention_by_frame_indices (wan_video_dit.py:85-128) multiplies 4-
// vectors of each head by per-frame camera matrices (prope_attention.py:
// 120-176): K and V by P^-1, Q by P^T, the output by P.  The fused camera
// kernel of the codec-native path (camera_kernel.py:8-36) rounds the matrix
// entries to bf16 and sums the four products in fp64; here likewise
// (the products are exact, the sum of four is exact in fp64), then
// fp64 -> fp32 -> bf16.
#pragma once

#include "nkv_common.h"

namespace nkv {

struct CameraDev {
    const float* mats = nullptr;  // [batches, n_mats, 4 sub-frames, 4, 4]; null: no camera
    int64_t mats_bs = 0;
    int n_mats = 0, layout = 0;
    const int32_t* frame_mat = nullptr;
    int64_t n_frames = 0;
    int tokens_per_frame = 1;
    // [launch heads, width / 8] sub-frame of each 8-dim block of a reader key
    // (camera_selected, CN/core.py:110-137), or null: the FULL/SF13 layout
    const int32_t* blocks = nullptr;
    // the matrices rounded to bf16, held in fp64, [mat batches, n_mats, 64]
    // (filled per call in the staged schedule's workspace), or null
    const double* m64 = nullptr;
};

// Matrix batches an nkv_camera holds for a call over B batch items.
__host__ __device__ __forceinline__ int camera_batches(const CameraDev& c, int B) {
    return c.mats_bs ? B : 1;
}

// Index of the matrix set of codec row `row` of batch item b (indices
// clamped), in units of one set (4 sub-frames x 16 entries).
__device__ __forceinline__ int64_t camera_set(const CameraDev& c, int b, int64_t row) {
    const int64_t f = min(max(row / c.tokens_per_frame, (int64_t)0), c.n_frames - 1);
    const int m = min(max(c.frame_mat[f], 0), c.n_mats - 1);
    return (c.mats_bs ? (int64_t)b * c.n_mats : 0) + m;
}

// Sub-frame matrices of codec row `row` of batch item b (indices clamped).
__device__ __forceinline__ const float* camera_mats(const CameraDev& c, int b, int64_t row) {
    const int64_t f = min(max(row / c.tokens_per_frame, (int64_t)0), c.n_frames - 1);
    const int m = min(max(c.frame_mat[f], 0), c.n_mats - 1);
    return c.mats + (int64_t)b * c.mats_bs + (int64_t)m * 64;
}

// y = bf16(M . x) for one 4-vector, M row-major 4x4 (fp32, used as bf16).
__device__ __forceinline__ void camera_vec4(const float* M, const float (&x)[4], float (&y)[4]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += (double)(bf16_round(M[4 * i + j]) * x[j]);
        y[i] = bf16_round(f64_to_f32(acc));
    }
}

// Output r of camera_vec4: bf16(M[r] . x), M row-major 4x4 (fp32, used as
// bf16).
__device__ __forceinline__ float camera_vec4_row(const float* M, int r, const float (&x)[4]) {
#pragma clang fp contract(off)
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += (double)(bf16_round(M[4 * r + j]) * x[j]);
    return bf16_round(f64_to_f32(acc));
}

// y = bf16(m . x) for one 4-vector, m row-major 4x4 already rounded to bf16.
__device__ __forceinline__ void camera_vec4_rounded(const float (&m)[16], const float (&x)[4],
                                                    float (&y)[4]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += (double)(m[4 * i + j] * x[j]);
        y[i] = bf16_round(f64_to_f32(acc));
    }
}

// The camera transform of one head row of D dims (D == 128 or the SF13
// layout) by the sub-frame matrices M (16-byte aligned), the row's dims read
// and written through get(d) / put(d, v).  Two lanes share a row: lane half
// hf takes every other 4-vector of each sub-frame, and each sub-frame's 16
// entries are loaded and rounded once.
template <int D, typename Get, typename Put>
__device__ __forceinline__ void camera_row(const float* M, int layout, int hf, Get get, Put put) {
    constexpr int RN = D / 64;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (layout && !(c & 1)) continue;  // SF13: sub-frames 1 and 3
        float m[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = reinterpret_cast<const float4*>(M + 16 * c)[q];
            m[4 * q] = bf16_round(f.x);
            m[4 * q + 1] = bf16_round(f.y);
            m[4 * q + 2] = bf16_round(f.z);
            m[4 * q + 3] = bf16_round(f.w);
        }
        const int nvec = layout ? 4 : 4 * RN;
        for (int k = hf; k < nvec; k += 2) {
            int base, step;
            if (layout) {
                base = (c == 1 ? 0 : 16) + 4 * k;
                step = 1;
            } else {
                base = ((k / RN) * 4 + c) * 4 * RN + k % RN;
                step = RN;
            }
            float x[4], y[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = get(base + j * step);
            camera_vec4_rounded(m, x, y);
#pragma unroll
            for (int j = 0; j < 4; ++j) put(base + j * step, y[j]);
        }
    }
}

// A head of D dims is D / 4 four-vectors; the dims of vector v: "full"
// (layout 0): d = ((p*4 + c)*4 + j)*rn + r (rn = D / 64), vector v = (p*4 +
// c)*rn + r over j, sub-frame c; "sf13" (layout 1): four contiguous dims per
// vector, sub-frame 1 on dims [0, 16), 3 on [16, 32), and sub = -1 (no
// transform) for the rest.
__host__ __device__ __forceinline__ int camera_vectors(int layout, int D) { return D / 4; }

__device__ __forceinline__ void camera_vector_dims(int layout, int D, int v, int& base, int& step,
                                                   int& sub) {
    if (layout) {
        base = 4 * v;
        step = 1;
        sub = v < 4 ? 1 : (v < 8 ? 3 : -1);
    } else {
        const int rn = D / 64;
        const int pc = v / rn, r = v % rn;
        base = pc * 4 * rn + r;
        step = rn;
        sub = pc % 4;
    }
}

// The camera transform of one reader row of W dims (W % 8 == 0) whose 8-dim
// block j uses sub-frame cams[j]: within a block the 4-vectors are dims
// {0, 2, 4, 6} and {1, 3, 5, 7} (the full layout's (j, r) order), so lane
// half hf takes vector hf of every block.  Each sub-frame's entries are
// loaded and rounded once per block.
template <int W, typename Get, typename Put>
__device__ __forceinline__ void camera_row_blocks(const float* M, const int32_t* cams, int hf,
                                                  Get get, Put put) {
#pragma unroll
    for (int j = 0; j < W / 8; ++j) {
        const int c = cams[j] & 3;
        float m[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = reinterpret_cast<const float4*>(M + 16 * c)[q];
            m[4 * q] = bf16_round(f.x);
            m[4 * q + 1] = bf16_round(f.y);
            m[4 * q + 2] = bf16_round(f.z);
            m[4 * q + 3] = bf16_round(f.w);
        }
        float x[4], y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = get(8 * j + 2 * e + hf);
        camera_vec4_rounded(m, x, y);
#pragma unroll
        for (int e = 0; e < 4; ++e) put(8 * j + 2 * e + hf, y[e]);
    }
}

// Host: validate an nkv_camera for heads of D dims and a call over B batch
// items, and fill dev (blocks stays null).
int camera_from_abi(const nkv_camera* c, int D, int B, CameraDev* dev);

// Host: x [B, S, H, D] bf16 times the camera in place (row s at codec row s),
// as nkv_camera_apply.
int camera_apply_inplace(hipStream_t s, const CameraDev& cam, int B, int64_t S, int H, int D,
                         uint16_t* x, int64_t sb, int64_t st, int64_t sh);

}  // namespace nkv
