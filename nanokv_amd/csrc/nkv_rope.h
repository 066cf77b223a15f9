// nkv_rope.h -- read-time rotary position embedding shared by the fused
// key-chunk kernel and nkv_rope_apply.
//
// rope_apply (wan_video_dit.py:185-192) multiplies each complex pair of a key
// by its position's frequency in fp64 and casts the result to bf16; the
// per-token frequencies are the concatenation of the temporal, row and
// column bands of precompute_freqs_cis_3d (wan_video_dit.py:168-182) as
// _kv_freqs (pipelines/wan_video.py:3322-3341) lays them out for frames of
// grid_h x grid_w tokens.  The bands stay separate here (a few KB each), and
// a key's codec row selects its entries.
#pragma once

#include "nkv_common.h"

namespace nkv {

struct RopeDev {
    const double* cs_t = nullptr;  // null: no RoPE
    const double* cs_h = nullptr;
    const double* cs_w = nullptr;
    const int32_t* frame_pos = nullptr;
    int64_t n_frames = 0;
    int n_t = 0, pt = 0, ph = 0, pw = 0, grid_h = 0, grid_w = 0;
    // [launch heads, width / 2] original pair of each pair of a narrower key
    // (rope_selected, CN/core.py:75-91), or null: pair j is pair j
    const int32_t* pairs = nullptr;
    // per-row table [n_rows, pt, 2] (pt = D / 2, ph = pw = 0), or null: bands
    const double* cs_rows = nullptr;
    int64_t n_rows = 0;
};

// Whether a RopeDev rotates anything.
__host__ __device__ __forceinline__ bool rope_on(const RopeDev& r) {
    return r.cs_t || r.cs_h || r.cs_w || r.cs_rows;
}

// The three band rows of one codec row (codec rows and the frame geometry
// are 32-bit, checked on the host); indices are clamped into the tables, so
// no row reads out of bounds.
struct RopeRows {
    const double* t;
    const double* h;
    const double* w;
};

__device__ __forceinline__ RopeRows rope_rows(const RopeDev& r, int64_t row64) {
    RopeRows rr;
    if (r.cs_rows) {
        // the whole row is the "temporal" band: pair p reads entry p
        rr.t = r.cs_rows + 2 * min(max(row64, (int64_t)0), r.n_rows - 1) * r.pt;
        rr.h = rr.w = rr.t;
        return rr;
    }
    const int tpf = r.grid_h * r.grid_w;
    const int row = (int)row64;
    const int f = row / tpf, rem = row - f * tpf, hr = rem / r.grid_w;
    rr.t = r.cs_t;
    if (r.pt) {
        const int tp = min(max(r.frame_pos[min(f, (int)r.n_frames - 1)], 0), r.n_t - 1);
        rr.t = r.cs_t + 2 * tp * r.pt;
    }
    rr.h = r.cs_h + 2 * hr * r.ph;
    rr.w = r.cs_w + 2 * (rem - hr * r.grid_w) * r.pw;
    return rr;
}

// (cos, sin) of pair p of a row (p is clamped into [0, pt + ph + pw))
__device__ __forceinline__ const double* rope_entry(const RopeDev& r, const RopeRows& rr, int p) {
    p = min(max(p, 0), r.pt + r.ph + r.pw - 1);
    return p < r.pt ? rr.t + 2 * p
                    : (p < r.pt + r.ph ? rr.h + 2 * (p - r.pt) : rr.w + 2 * (p - r.pt - r.ph));
}

// Rotate the bf16 pair (lo, hi) of `w` by (c, s) in fp64, every product and
// sum rounded (no fused multiply-add, whatever the translation unit's
// contraction policy), then fp64 -> fp32 -> bf16.
__device__ __forceinline__ uint32_t rope_pair(uint32_t w, double c, double s) {
#pragma clang fp contract(off)
    const double a = (double)__uint_as_float(w << 16);
    const double b = (double)__uint_as_float(w & 0xffff0000u);
    // (HIP's __dmul_rn is a plain product the translation unit may contract;
    // the pragma above holds for these operations)
    const double ac = a * c, bs = b * s, as = a * s, bc = b * c;
    const float y0 = f64_to_f32(ac - bs);
    const float y1 = f64_to_f32(as + bc);
    return pack_bf16x2(y0, y1);
}

// Host: validate an nkv_rope for heads of D dims (D / 2 pairs) and fill dev
// (pairs stays null).  Returns NKV_OK or an error code with the message set.
int rope_from_abi(const nkv_rope* r, int D, RopeDev* dev);

// Host: rows an nkv_rope gives positions to (its per-row table, or its frames).
inline int64_t rope_rows_covered(const nkv_rope* r) {
    return r->cs_rows ? r->n_rows : r->n_frames * (int64_t)r->grid_h * r->grid_w;
}

}  // namespace nkv
