// nkv_rope.hip -- RoPE of bf16 rows at codec-row positions (nkv_rope_apply)
// and the validation of nkv_rope shared with nkv_attend.
//
// Restates rope_apply (wan_video_dit.py:185-192): x in fp64, times the
// position's complex frequency, cast to bf16; the frequency of pair p comes
// from one of three bands (nkv_rope.h).  Memory-bound: one thread rotates
// PPT pairs of one (b, s, h) row with one load and one store of x.
#include "nkv_rope.h"

#include "nkv_internal.h"

namespace nkv {

int rope_from_abi(const nkv_rope* r, int D, RopeDev* dev) {
    NKV_REQUIRE(r, NKV_ERR_INVALID, "rope is null");
    NKV_REQUIRE(D > 0 && D % 2 == 0, NKV_ERR_INVALID, "RoPE needs an even head dimension");
    if (r->cs_rows) {
        NKV_REQUIRE(r->n_rows >= 1, NKV_ERR_INVALID, "a per-row RoPE table needs n_rows >= 1");
        *dev = RopeDev{};
        dev->cs_rows = r->cs_rows;
        dev->n_rows = r->n_rows;
        dev->pt = D / 2;
        return NKV_OK;
    }
    NKV_REQUIRE(r->pt >= 0 && r->ph >= 0 && r->pw >= 0 && r->pt + r->ph + r->pw == D / 2,
                NKV_ERR_INVALID, "RoPE bands must hold D / 2 pairs (pt + ph + pw)");
    NKV_REQUIRE(r->grid_h >= 1 && r->grid_w >= 1 && r->n_frames >= 1, NKV_ERR_INVALID,
                "RoPE needs grid_h, grid_w and n_frames >= 1");
    NKV_REQUIRE(r->pt == 0 || (r->cs_t && r->frame_pos && r->n_t >= 1), NKV_ERR_INVALID,
                "RoPE temporal band needs cs_t, frame_pos and n_t >= 1");
    NKV_REQUIRE(r->ph == 0 || r->cs_h, NKV_ERR_INVALID, "RoPE row band needs cs_h");
    NKV_REQUIRE(r->n_frames * (int64_t)r->grid_h * r->grid_w < INT32_MAX, NKV_ERR_INVALID,
                "RoPE frames must cover fewer than 2^31 rows");
    NKV_REQUIRE(r->pw == 0 || r->cs_w, NKV_ERR_INVALID, "RoPE column band needs cs_w");
    dev->cs_t = r->cs_t;
    dev->cs_h = r->cs_h;
    dev->cs_w = r->cs_w;
    dev->frame_pos = r->frame_pos;
    dev->n_frames = r->n_frames;
    dev->n_t = r->n_t;
    dev->pt = r->pt;
    dev->ph = r->ph;
    dev->pw = r->pw;
    dev->grid_h = r->grid_h;
    dev->grid_w = r->grid_w;
    dev->pairs = nullptr;
    return NKV_OK;
}

namespace {

struct RopeApplyParams {
    RopeDev rope;
    int B, H, D;
    int64_t S;
    const uint16_t* x;
    int64_t x_sb, x_st, x_sh;
    const int32_t* rows;
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
};

// PPT pairs per thread: 4 (16-byte accesses, D % 8 == 0) or 1
template <int PPT>
__global__ void __launch_bounds__(256) rope_apply_kernel(RopeApplyParams p) {
    const int per_row = p.D / (2 * PPT);
    const int64_t total = (int64_t)p.B * p.S * p.H * per_row;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int part = (int)(i % per_row);
        int64_t rest = i / per_row;
        const int h = (int)(rest % p.H);
        rest /= p.H;
        const int64_t s = rest % p.S;
        const int b = (int)(rest / p.S);
        const RopeRows rr = rope_rows(p.rope, p.rows ? (int64_t)p.rows[s] : s);
        const uint16_t* src = p.x + b * p.x_sb + s * p.x_st + h * p.x_sh + 2 * PPT * part;
        uint16_t* dst = p.out + b * p.o_sb + s * p.o_st + h * p.o_sh + 2 * PPT * part;
        if constexpr (PPT == 4) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(src);
            u32x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double* cs = rope_entry(p.rope, rr, 4 * part + e);
                y[e] = rope_pair(w[e], cs[0], cs[1]);
            }
            *reinterpret_cast<u32x4*>(dst) = y;
        } else {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
            const double* cs = rope_entry(p.rope, rr, part);
            *reinterpret_cast<uint32_t*>(dst) = rope_pair(w, cs[0], cs[1]);
        }
    }
}

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int nkv_rope_apply(void* stream, const nkv_rope* rope, int B, int64_t S, int H, int D,
                              const uint16_t* x, int64_t x_sb, int64_t x_st, int64_t x_sh,
                              const int32_t* rows, uint16_t* out, int64_t o_sb, int64_t o_st,
                              int64_t o_sh) {
    clear_error();
    RopeApplyParams p;
    int rc = rope_from_abi(rope, D, &p.rope);
    if (rc) return rc;
    NKV_REQUIRE(B >= 0 && S >= 0 && H >= 0, NKV_ERR_INVALID, "negative shape");
    if ((int64_t)B * S * H == 0) return NKV_OK;
    NKV_REQUIRE(x && out, NKV_ERR_INVALID, "x and out are required");
    NKV_REQUIRE(rows || S <= rope_rows_covered(rope), NKV_ERR_INVALID,
                "more rows than the RoPE frames cover");
    NKV_REQUIRE(S < INT32_MAX, NKV_ERR_INVALID, "RoPE rows must fit in 32 bits");
    const bool vec = D % 8 == 0 && (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0 &&
                     x_sb % 8 == 0 && x_st % 8 == 0 && x_sh % 8 == 0 && o_sb % 8 == 0 &&
                     o_st % 8 == 0 && o_sh % 8 == 0;
    p.B = B;
    p.H = H;
    p.D = D;
    p.S = S;
    p.x = x;
    p.x_sb = x_sb;
    p.x_st = x_st;
    p.x_sh = x_sh;
    p.rows = rows;
    p.out = out;
    p.o_sb = o_sb;
    p.o_st = o_st;
    p.o_sh = o_sh;
    const int64_t items = (int64_t)B * S * H * (D / (vec ? 8 : 2));
    const unsigned grid = (unsigned)std::min<int64_t>(cdiv(items, 256), 65536);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (vec)
        rope_apply_kernel<4><<<grid, 256, 0, s>>>(p);
    else
        rope_apply_kernel<1><<<grid, 256, 0, s>>>(p);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
