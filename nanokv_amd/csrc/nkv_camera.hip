// nkv_camera.hip -- camera PRoPE transform of bf16 rows (nkv_camera_apply) and
// the validation of nkv_camera shared with nkv_attend.
//
// One thread per (b, s, h, 4-vector): load its four dims, multiply by the
// sub-frame matrix of the row's frame (nkv_camera.h), store.
#include "nkv_camera.h"

#include "nkv_internal.h"

namespace nkv {

int camera_from_abi(const nkv_camera* c, int D, int B, CameraDev* dev) {
    NKV_REQUIRE(c, NKV_ERR_INVALID, "camera is null");
    NKV_REQUIRE(c->mats && c->frame_mat, NKV_ERR_INVALID, "camera needs mats and frame_mat");
    NKV_REQUIRE(c->n_mats >= 1 && c->n_frames >= 1 && c->tokens_per_frame >= 1 && c->mats_bs >= 0,
                NKV_ERR_INVALID, "camera needs n_mats, n_frames, tokens_per_frame >= 1");
    NKV_REQUIRE(((uintptr_t)c->mats & 15) == 0 && c->mats_bs % 4 == 0, NKV_ERR_INVALID,
                "camera mats must be 16-byte aligned (mats_bs a multiple of 4)");
    NKV_REQUIRE(c->layout == NKV_CAMERA_FULL || c->layout == NKV_CAMERA_SF13, NKV_ERR_INVALID,
                "unknown camera layout");
    NKV_REQUIRE(c->layout != NKV_CAMERA_FULL || (D > 0 && D % 64 == 0), NKV_ERR_INVALID,
                "the FULL camera layout needs D % 64 == 0");
    NKV_REQUIRE(c->layout != NKV_CAMERA_SF13 || D >= 32, NKV_ERR_INVALID,
                "the SF13 camera layout needs D >= 32");
    NKV_REQUIRE(c->mats_bs == 0 || B <= c->n_batches, NKV_ERR_INVALID,
                "camera mats hold fewer matrix batches than the call's batch items");
    dev->mats = c->mats;
    dev->mats_bs = c->mats_bs;
    dev->n_mats = c->n_mats;
    dev->layout = c->layout;
    dev->frame_mat = c->frame_mat;
    dev->n_frames = c->n_frames;
    dev->tokens_per_frame = c->tokens_per_frame;
    dev->blocks = nullptr;
    return NKV_OK;
}

namespace {

struct CameraApplyParams {
    CameraDev cam;
    int B, H, D;
    int64_t S;
    const uint16_t* x;
    int64_t x_sb, x_st, x_sh;
    const int32_t* rows;
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
};

__global__ void __launch_bounds__(256) camera_apply_kernel(CameraApplyParams p) {
    const int nv = camera_vectors(p.cam.layout, p.D);
    const int64_t total = (int64_t)p.B * p.S * p.H * nv;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int v = (int)(i % nv);
        int64_t rest = i / nv;
        const int h = (int)(rest % p.H);
        rest /= p.H;
        const int64_t s = rest % p.S;
        const int b = (int)(rest / p.S);
        const int64_t row = p.rows ? (int64_t)p.rows[s] : s;
        int base, step, sub;
        camera_vector_dims(p.cam.layout, p.D, v, base, step, sub);
        const uint16_t* src = p.x + b * p.x_sb + s * p.x_st + h * p.x_sh + base;
        uint16_t* dst = p.out + b * p.o_sb + s * p.o_st + h * p.o_sh + base;
        if (sub < 0) {  // dims the layout leaves alone
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j * step] = src[j * step];
            continue;
        }
        float x[4], y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = bf16_bits_to_f32(src[j * step]);
        camera_vec4(camera_mats(p.cam, b, row) + 16 * sub, x, y);
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[j * step] = f32_to_bf16_bits(y[j]);
    }
}

}  // namespace
}  // namespace nkv

using namespace nkv;

namespace nkv {

int camera_apply_inplace(hipStream_t s, const CameraDev& cam, int B, int64_t S, int H, int D,
                         uint16_t* x, int64_t sb, int64_t st, int64_t sh) {
    if ((int64_t)B * S * H == 0) return NKV_OK;
    CameraApplyParams p;
    p.cam = cam;
    p.B = B;
    p.H = H;
    p.D = D;
    p.S = S;
    p.x = x;
    p.x_sb = sb;
    p.x_st = st;
    p.x_sh = sh;
    p.rows = nullptr;
    p.out = x;
    p.o_sb = sb;
    p.o_st = st;
    p.o_sh = sh;
    const int64_t items = (int64_t)B * S * H * camera_vectors(cam.layout, D);
    const unsigned grid = (unsigned)std::min<int64_t>(cdiv(items, 256), 65536);
    camera_apply_kernel<<<grid, 256, 0, s>>>(p);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

}  // namespace nkv

extern "C" int nkv_camera_apply(void* stream, const nkv_camera* camera, int B, int64_t S, int H,
                                int D, const uint16_t* x, int64_t x_sb, int64_t x_st,
                                int64_t x_sh, const int32_t* rows, uint16_t* out, int64_t o_sb,
                                int64_t o_st, int64_t o_sh) {
    clear_error();
    CameraApplyParams p;
    int rc = camera_from_abi(camera, D, B, &p.cam);
    if (rc) return rc;
    NKV_REQUIRE(B >= 0 && S >= 0 && H >= 0, NKV_ERR_INVALID, "negative shape");
    if ((int64_t)B * S * H == 0) return NKV_OK;
    NKV_REQUIRE(x && out, NKV_ERR_INVALID, "x and out are required");
    NKV_REQUIRE(D % 4 == 0, NKV_ERR_INVALID, "D must be a multiple of 4");
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
    const int64_t items = (int64_t)B * S * H * camera_vectors(camera->layout, D);
    const unsigned grid = (unsigned)std::min<int64_t>(cdiv(items, 256), 65536);
    camera_apply_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(p);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
