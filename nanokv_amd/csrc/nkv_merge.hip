// nkv_merge.hip -- output merges of the Fast partitions of the HY and
// LingBot backbones (gfx950): HY's value lift of its two history branches
// fused with the LSE merge into the native output (nkv_lift_lse_combine), and
// LingBot's finish of one reader group with its value-mean correction and
// head scatter (nkv_finish).  Both are bandwidth-bound epilogues: each output
// element is read once from every input and written once.  Compiled without
// FMA contraction, as the reference kernels are (enable_fp_fusion=False).
#include "nkv_common.h"
#include "nkv_internal.h"

namespace nkv {

namespace {

// ---- nkv_lift_lse_combine (HYP:883-1014)
// One block per (32 queries, batch item b of 2B, head h).  The block's low
// rows and the head's lift (Main [low_dim, 128], or PRoPE mix [low_dim/4, 32])
// are staged in LDS as fp32; thread t computes output column t % 128 of
// queries t / 128, t / 128 + 2, ...  Each output is a sum of bf16 products
// in fp32 (the lift of one low row), merged with the native value by the two
// LSEs.
constexpr int LC_Q = 32;
constexpr int LC_THREADS = 256;
constexpr int LC_MAXK = 96;

__global__ void __launch_bounds__(LC_THREADS) lift_combine_kernel(nkv_lift_combine_args a) {
    __shared__ float low[LC_Q][LC_MAXK + 1];
    __shared__ float w[LC_MAXK * 128];
    const int t = threadIdx.x;
    const int64_t q0 = (int64_t)blockIdx.x * LC_Q;
    const int b = (int)(blockIdx.y / a.H), h = (int)(blockIdx.y % a.H);
    const bool prope = b >= a.B;
    const int K = a.low_dim;
    for (int i = t; i < LC_Q * K; i += LC_THREADS) {
        const int q = i / K, k = i % K;
        const int64_t qi = q0 + q;
        low[q][k] = qi < a.Q ? bf16_bits_to_f32(a.low[b * a.l_sb + h * a.l_sh + qi * a.l_sq +
                                                      k * a.l_sd])
                             : 0.0f;
    }
    if (!prope) {
        for (int i = t; i < K * 128; i += LC_THREADS) {
            const int k = i >> 7, o = i & 127;
            w[i] = bf16_bits_to_f32(a.main_lift[h * a.ml_sh + k * a.ml_sk + o * a.ml_so]);
        }
    } else {
        for (int i = t; i < (K / 4) * 32; i += LC_THREADS) {
            const int k = i >> 5, j = i & 31;
            w[i] = bf16_bits_to_f32(a.prope_mix[h * a.pm_sh + k * a.pm_sk + j * a.pm_so]);
        }
    }
    __syncthreads();
    const int o = t & 127;
    for (int q = t >> 7; q < LC_Q; q += LC_THREADS / 128) {
        const int64_t qi = q0 + q;
        if (qi >= a.Q) break;
        float acc = 0.0f;
        if (!prope) {
            for (int k = 0; k < K; ++k) acc += low[q][k] * w[k * 128 + o];
        } else {
            // output dim 4 j + c of coordinate c takes quartets k of low dim 4 k + c
            const int c = o & 3, j = o >> 2;
            for (int k = 0; k < K / 4; ++k) acc += low[q][4 * k + c] * w[k * 32 + j];
        }
        const float x = a.native_lse[b * a.nl_sb + h * a.nl_sh + qi * a.nl_sq];
        const float y = a.history_lse[b * a.hl_sb + h * a.hl_sh + qi * a.hl_sq];
        const float m = fmaxf(x, y);
        const float wn = expf(x - m), wh = expf(y - m);
        const float nv =
            bf16_bits_to_f32(a.native[b * a.n_sb + h * a.n_sh + qi * a.n_sq + o * a.n_sd]);
        a.out[(((int64_t)b * a.H + h) * a.Q + qi) * 128 + o] =
            f32_to_bf16_bits((nv * wn + acc * wh) / (wn + wh));
    }
}

// ---- nkv_finish (LBF:10-34)
// One wave per (b, group head g, s) row; lanes stride over d.  Each lane
// reads its elements' native values before it writes them, so result may
// alias native.
constexpr int FN_WAVES = 4;

__global__ void __launch_bounds__(64 * FN_WAVES) finish_kernel(nkv_finish_args a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * FN_WAVES + (threadIdx.x >> 6);
    const int64_t rows = (int64_t)a.B * a.H_group * a.S;
    if (row >= rows) return;
    const int64_t s = row % a.S;
    const int g = (int)((row / a.S) % a.H_group);
    const int b = (int)(row / ((int64_t)a.S * a.H_group));
    const int hd = a.heads[g];
    // a head index outside the native heads (a corrupt map) writes nothing
    if (hd < 0 || hd >= a.H_native) return;
    const float x = a.native_lse[b * a.la_sb + hd * a.la_sh + s * a.la_ss];
    const float z = a.low_lse[b * a.lb_sb + g * a.lb_sh + s * a.lb_ss];
    float l = fmaxf(x, z) + log1pf(expf(-fabsf(x - z)));
    if (x == z && fabsf(x) == INFINITY) l = x;
    const float origin = fabsf(l) != INFINITY ? l : 0.0f;
    const float ea = expf(x - origin), eb = expf(z - origin);
    const bool correct = a.mean != nullptr;
    const uint16_t* arow = a.native + b * a.a_sb + hd * a.a_sh + s * a.a_ss;
    const uint16_t* brow = a.lifted + b * a.b_sb + g * a.b_sh + s * a.b_ss;
    uint16_t* yrow = a.result + b * a.y_sb + hd * a.y_sh + s * a.y_ss;
    for (int d = lane; d < a.D; d += 64) {
        const float av = bf16_bits_to_f32(arow[d * a.a_sd]);
        float bv = bf16_bits_to_f32(brow[d * a.b_sd]);
        if (correct)
            bv = (bv + a.mean[b * a.m_sb + hd * a.m_sh + d * a.m_sd]) -
                 a.projected[b * a.p_sb + g * a.p_sh + d * a.p_sd];
        yrow[d * a.y_sd] = f32_to_bf16_bits(av * ea + bv * eb);
    }
}

}  // namespace

}  // namespace nkv

using namespace nkv;

extern "C" int nkv_lift_lse_combine(void* stream, const nkv_lift_combine_args* a) {
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null arguments");
    NKV_REQUIRE(a->B >= 0 && a->H >= 1 && a->Q >= 0, NKV_ERR_INVALID, "bad shape");
    NKV_REQUIRE(a->low_dim == 32 || a->low_dim == 64 || a->low_dim == 96, NKV_ERR_UNSUPPORTED,
                "the fused lift supports low_dim 32, 64 and 96");
    if (a->B == 0 || a->Q == 0) return NKV_OK;
    NKV_REQUIRE(a->native && a->native_lse && a->low && a->main_lift && a->prope_mix &&
                    a->history_lse && a->out,
                NKV_ERR_INVALID, "null pointer");
    const int64_t heads = 2 * (int64_t)a->B * a->H;
    NKV_REQUIRE(heads <= 65535, NKV_ERR_UNSUPPORTED, "at most 65535 batch x head pairs");
    lift_combine_kernel<<<dim3((unsigned)cdiv(a->Q, LC_Q), (unsigned)heads), LC_THREADS, 0,
                          (hipStream_t)stream>>>(*a);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

extern "C" int nkv_finish(void* stream, const nkv_finish_args* a) {
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null arguments");
    NKV_REQUIRE(a->B >= 0 && a->H_native >= 1 && a->H_group >= 0 && a->S >= 0 && a->D >= 1,
                NKV_ERR_INVALID, "bad shape");
    NKV_REQUIRE((a->mean == nullptr) == (a->projected == nullptr), NKV_ERR_INVALID,
                "mean and projected come together (the value-mean correction) or not at all");
    const int64_t rows = (int64_t)a->B * a->H_group * a->S;
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(a->native && a->native_lse && a->lifted && a->low_lse && a->heads && a->result,
                NKV_ERR_INVALID, "null pointer");
    finish_kernel<<<dim3((unsigned)cdiv(rows, FN_WAVES)), 64 * FN_WAVES, 0, (hipStream_t)stream>>>(
        *a);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
