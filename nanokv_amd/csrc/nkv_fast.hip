// nkv_fast.hip -- NanoKV-Fast mixed-dimensional history attention for gfx950
// (nkv_fast_attend): hybrid_attention (CN/core.py:278-310) with the partition
// reads of maybe_attention (CN/mg35.py:100-357), fused per partition.
// With RoPE, the history keys of both partitions are rotated in-kernel after
// decode (the low partition on the reader's retained pairs) and the reader
// queries are formed from the pre-RoPE queries and rotated likewise
// (CN/mg35.py:207-214, 305-336).
//
// Per layer call:
//  1. native partition: every head attends its queries to the protected
//     history rows (decoded in-kernel at full width, as nkv_attend does) and
//     the current keys -> out (bf16) and lse_n (CN/mg35.py:192-303);
//  2. per reader group (CN/core.py:155-204), for its heads:
//       q_low   = bf16(q . q_reduce)                          (query, :164-166)
//       centers = bf16(center columns . affine), bias = bf16(bf16(mean) . affine)
//       k_low   = bf16(bf16(latent . k_read^T + bias) + centers[id])  (read, :168-200)
//       v_low   likewise with v_read / v_affine (width D)
//     the low rows are attended by the same key-chunk kernel at K/Q width d,
//     decoding k_low / v_low in-kernel -> out_l, lse_l;
//  3. merge(out, lse_n, out_l, lse_l) per group head (CN/core.py:33-42), the
//     lift being the identity (vd == D).
// With at most NKV_MAX_PARTS - 1 groups, all partitions run as one staged
// launch (staged_multi_launch): one decode launch for every partition's
// tiles, with read-time RoPE or the camera one in-place pass over them,
// one flash launch over all of them, and one combine that folds each head's
// native and group partials together (the merge of step 3, with the
// low_shift), so no group output or LSE is written.  Identity readers then
// read the layer's own center tables and means (and, without RoPE or the
// camera, queries) through head maps instead of projected copies.  Otherwise the partitions run one after another and
// group_merge_kernel merges each group's output in place.
// The projected tables are small (C x d per head); they are recomputed per
// call, as the reference's read does.  With a segmented codec the tables of
// every segment are projected into one table (segment s at rows center_base
// ..) in one launch, and the low launch reads row center_base + id.
// Camera (CN/mg35.py:253-257, 310-346): the history rows of both partitions
// are multiplied by P^-1 in-kernel (the reader keys on their own 8-dim
// blocks, camera_selected CN/core.py:110-137), q_low by P^T of the query
// rows; the value lift is folded into the value reader, so the values and
// the output stay in the native layout and the caller applies P to out.
#include "nkv_common.h"
#include "nkv_internal.h"

#include <vector>

namespace nkv {

// Source row (b, m, head) of a projection: x[b*x_b + m*x_m + head*x_h], or,
// with a segment table, row m of the concatenation of the segments' center
// tables (segment s holds rows center_base .. center_base + num_centers).
template <bool X_F32>
__device__ __forceinline__ const void* proj_row(const void* x, int64_t x_b, int64_t x_m, int64_t x_h,
                                                const nkv_segment* seg, int n_seg, int b, int64_t m,
                                                int head) {
    if (seg) {
        int lo = 0, hi = n_seg - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (seg[mid].center_base <= m) lo = mid;
            else hi = mid - 1;
        }
        const nkv_segment& sg = seg[lo];
        const int64_t local = min(max(m - sg.center_base, (int64_t)0), (int64_t)sg.num_centers - 1);
        return sg.centers + (int64_t)b * sg.centers_batch_stride + local * x_m + (int64_t)head * x_h;
    }
    const int64_t off = (int64_t)b * x_b + m * x_m + (int64_t)head * x_h;
    return X_F32 ? (const void*)(reinterpret_cast<const float*>(x) + off)
                 : (const void*)(reinterpret_cast<const uint16_t*>(x) + off);
}

// out[b][i][m][e] = bf16(sum_d x(b, m, heads[i], d) * w[i][d][e]) with
// x(b, m, h, d) = x[b*x_b + m*x_m + h*x_h + d] (bf16 bits, or fp32 rounded to
// bf16 first when X_F32), w == null meaning the identity (E == D).  The
// output element is stored at out[b*o_b + i*o_i + m*o_m + e]; OUT_F32 stores
// the bf16-rounded value as fp32.  One thread per output element, fp32
// accumulation.  seg: rows come from the segments' center tables (proj_row).
template <bool X_F32, bool OUT_F32>
__global__ void __launch_bounds__(256) project_kernel(const void* x, int64_t x_b, int64_t x_m,
                                                      int64_t x_h, const nkv_segment* seg,
                                                      int n_seg, const int32_t* heads, int H,
                                                      const uint16_t* w, int D, int E, int nb,
                                                      int nh, int64_t M, void* out, int64_t o_b,
                                                      int64_t o_i, int64_t o_m) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)nb * nh * M * E;
    if (tid >= total) return;
    const int e = (int)(tid % E);
    int64_t r = tid / E;
    const int64_t m = r % M;
    r /= M;
    const int i = (int)(r % nh);
    const int b = (int)(r / nh);
    // head indices outside the layer are clamped (no out-of-bounds reads)
    const void* xr = proj_row<X_F32>(x, x_b, x_m, x_h, seg, n_seg, b, m, min(max(heads[i], 0), H - 1));
    float acc;
    if (w == nullptr) {
        acc = X_F32 ? bf16_round(reinterpret_cast<const float*>(xr)[e])
                    : bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(xr)[e]);
    } else {
        acc = 0.0f;
        const uint16_t* wi = w + (int64_t)i * D * E + e;
        for (int d = 0; d < D; ++d) {
            const float xv = X_F32 ? bf16_round(reinterpret_cast<const float*>(xr)[d])
                                   : bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(xr)[d]);
            acc = fmaf(xv, bf16_bits_to_f32(wi[(int64_t)d * E]), acc);
        }
    }
    const int64_t o = (int64_t)b * o_b + (int64_t)i * o_i + m * o_m + e;
    if (OUT_F32) reinterpret_cast<float*>(out)[o] = bf16_round(acc);
    else reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16_bits(acc);
}

// The same projection on MFMA for a non-identity w (D <= 128, E in {32, 64,
// 128}): a block owns 128 rows m of one (b, i) and all E columns; w[i] is
// staged transposed in LDS ([e][d], 16-byte operand reads) and each wave
// computes 32 rows x E with v_mfma_f32_32x32x16_bf16.  The bf16 rounding of
// the inputs and of the fp32 sum is that of project_kernel; only the order
// of the fp32 sum differs.
constexpr int PJ_ROWS = 128, PJ_MAXE = 128, PJ_MAXD = 128, PJ_PAD = 8;

template <bool X_F32, bool OUT_F32>
__global__ void __launch_bounds__(256) project_mfma_kernel(const void* x, int64_t x_b, int64_t x_m,
                                                           int64_t x_h, const nkv_segment* seg,
                                                           int n_seg, const int32_t* heads, int H,
                                                           const uint16_t* w, int D, int E,
                                                           int64_t M, void* out, int64_t o_b,
                                                           int64_t o_i, int64_t o_m) {
    __shared__ __align__(16) uint16_t wt[PJ_MAXE][PJ_MAXD + PJ_PAD];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    const int i = blockIdx.y, b = blockIdx.z;
    const uint16_t* wi = w + (int64_t)i * D * E;
    for (int idx = t; idx < D * E; idx += 256) wt[idx % E][idx / E] = wi[idx];
    __syncthreads();
    const int64_t m = (int64_t)blockIdx.x * PJ_ROWS + 32 * wave + l32;
    const int64_t ml = m < M ? m : M - 1;  // rows past the end read the last row (not stored)
    const void* xr =
        proj_row<X_F32>(x, x_b, x_m, x_h, seg, n_seg, b, ml, min(max(heads[i], 0), H - 1));
    const int ntile = E / 32;
    f32x16 acc[PJ_MAXE / 32];
#pragma unroll
    for (int tt = 0; tt < PJ_MAXE / 32; ++tt) acc[tt] = f32x16{};
    for (int k0 = 0; k0 < D; k0 += 16) {
        u32x4 a;
        if (X_F32) {
            const float* xp = reinterpret_cast<const float*>(xr) + k0 + 8 * hf;
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(xp);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(xp + 4);
            a = u32x4{pack_bf16x2(x0[0], x0[1]), pack_bf16x2(x0[2], x0[3]),
                      pack_bf16x2(x1[0], x1[1]), pack_bf16x2(x1[2], x1[3])};
        } else {
            a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(xr) + k0 + 8 * hf);
        }
#pragma unroll
        for (int tt = 0; tt < PJ_MAXE / 32; ++tt)
            if (tt < ntile)
                acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    as_bf16x8(a), *reinterpret_cast<const bf16x8*>(&wt[32 * tt + l32][k0 + 8 * hf]),
                    acc[tt], 0, 0, 0);
    }
#pragma unroll
    for (int tt = 0; tt < PJ_MAXE / 32; ++tt) {
        if (tt >= ntile) continue;
        const int e = 32 * tt + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t mr = (int64_t)blockIdx.x * PJ_ROWS + 32 * wave + 8 * (r / 4) + 4 * hf + (r % 4);
            if (mr >= M) continue;
            const int64_t o = (int64_t)b * o_b + (int64_t)i * o_i + mr * o_m + e;
            if (OUT_F32) reinterpret_cast<float*>(out)[o] = bf16_round(acc[tt][r]);
            else reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16_bits(acc[tt][r]);
        }
    }
}

// Merge of each group head's native and low partitions, in place in out
// (CN/core.py:33-42): lse = logaddexp(la, lb); origin = lse if finite else
// 0; out = a e^(la - origin) + b e^(lb - origin) in fp32, rounded to bf16.
// Sixteen threads per (b, q, i) row of D = 128 values, 8 values (16 bytes)
// each.
__global__ void __launch_bounds__(256) group_merge_kernel(
    int B, int64_t Q, int nh, int D, const int32_t* heads, uint16_t* out, int64_t o_sb,
    int64_t o_st, int64_t o_sh, const float* lse_n, int H, const uint16_t* low, const float* lse_l,
    float* lse_out, const float* shift, int64_t sh_sb, int64_t sh_sh) {
    const int per_row = D / 8;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= (int64_t)B * Q * nh * per_row) return;
    const int part = (int)(tid % per_row);
    const int64_t row = tid / per_row;
    const int i = (int)(row % nh);
    const int64_t q = (row / nh) % Q;
    const int b = (int)(row / ((int64_t)nh * Q));
    const int h = min(max(heads[i], 0), H - 1);
    const float x = lse_n[((int64_t)b * H + h) * Q + q];
    const float y = lse_l[((int64_t)b * nh + i) * Q + q];
    // logaddexp: max + log1p(exp(-|x - y|)); equal inputs (including -inf) give x + ln 2
    const float l = x == y ? x + 0.69314718055994531f : fmaxf(x, y) + log1pf(expf(-fabsf(x - y)));
    const float origin = isfinite(l) ? l : 0.0f;
    const float wa = expf(x - origin), wb = expf(y - origin);
    u32x4* op = reinterpret_cast<u32x4*>(out + (int64_t)b * o_sb + q * o_st + (int64_t)h * o_sh + 8 * part);
    const u32x4 lv = *reinterpret_cast<const u32x4*>(low + (((int64_t)b * Q + q) * nh + i) * D + 8 * part);
    const u32x4 ov = *op;
    // the value-mean correction shifts the low output of head h
    float sv[8] = {};
    if (shift) {
        const float* sp = shift + (int64_t)b * sh_sb + (int64_t)h * sh_sh + 8 * part;
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = sp[e];
    }
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        r[e] = pack_bf16x2(
            __uint_as_float(ov[e] << 16) * wa + (__uint_as_float(lv[e] << 16) + sv[2 * e]) * wb,
            __uint_as_float(ov[e] & 0xffff0000u) * wa +
                (__uint_as_float(lv[e] & 0xffff0000u) + sv[2 * e + 1]) * wb);
    *op = r;
    if (lse_out && part == 0) lse_out[((int64_t)b * H + h) * Q + q] = l;
}

// The reader queries' read-time transforms in one pass over up to QL_MAX
// reader groups: q_low [B, Q, nh, d] bf16 of each group written in place, or
// from the layer's queries src[b, t, heads[i]] (an identity q_reduce, d ==
// D) when the group's src is given.  RoPE rotates pair p of head i by
// original pair pairs[i * d/2 + p] (null: p) at the position of query t
// (rope_selected, CN/core.py:75-91), then the camera multiplies the two
// 4-vectors of 8-dim block j -- its dims {0, 2, 4, 6} and {1, 3, 5, 7} -- by
// sub-frame cams[i * d/8 + j] (null: j % 4) of query t's matrices
// (camera_selected, CN/core.py:110-137).  One thread per (group, b, t, i,
// block): one 16-byte load and store.
constexpr int QL_MAX = 8;
struct QueryLowGroup {
    uint16_t* q_low;
    const uint16_t* src;
    const int32_t* heads;
    const int32_t* pairs;
    const int32_t* cams;
    int nh, d;
    int ostride;   // elements per q_low row (>= d; the columns past d are zeroed)
};
struct QueryLowBatch {
    QueryLowGroup g[QL_MAX];
    int64_t first[QL_MAX + 1];  // first thread of each group
    int n, H, B;
    int64_t Q, s_b, s_t, s_h;
    RopeDev pos;
    CameraDev cam;
};

__global__ void __launch_bounds__(256) query_low_kernel(QueryLowBatch P) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gt >= P.first[P.n]) return;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < QL_MAX; ++i)
        if (i < P.n && gt >= P.first[i]) gi = i;
    const QueryLowGroup& G = P.g[gi];
    const int64_t tid = gt - P.first[gi];
    const int nbk = G.d / 8, nunit = G.ostride / 8;
    const int j = (int)(tid % nunit);
    const int64_t row = tid / nunit;  // (b, t, i)
    const int i = (int)(row % G.nh);
    const int64_t t = (row / G.nh) % P.Q;
    const int b = (int)(row / ((int64_t)G.nh * P.Q));
    uint16_t* dst = G.q_low + row * G.ostride + 8 * j;
    if (j >= nbk) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    const uint16_t* from = dst;
    if (G.src) {
        const int hq = min(max(ldg(G.heads + i), 0), P.H - 1);
        from = G.src + b * P.s_b + t * P.s_t + hq * P.s_h + 8 * j;
    }
    u32x4 v = ldg(reinterpret_cast<const u32x4*>(from));
    if (rope_on(P.pos)) {
        const RopeRows rr = rope_rows(P.pos, t);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int pj = G.pairs ? ldg(G.pairs + (int64_t)i * (G.d / 2) + 4 * j + w) : 4 * j + w;
            const f64x2 cs = ldg(reinterpret_cast<const f64x2*>(rope_entry(P.pos, rr, pj)));
            v[w] = rope_pair(v[w], cs.x, cs.y);
        }
    }
    if (P.cam.mats) {
        const int sub = G.cams ? (ldg(G.cams + (int64_t)i * nbk + j) & 3) : (j & 3);
        const float* M = camera_mats(P.cam, b, t) + 16 * sub;
        float x0[4], x1[4], y0[4], y1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x0[e] = __uint_as_float(v[e] << 16);
            x1[e] = __uint_as_float(v[e] & 0xffff0000u);
        }
        camera_vec4(M, x0, y0);
        camera_vec4(M, x1, y1);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = pack_bf16x2(y0[e], y1[e]);
    }
    *reinterpret_cast<u32x4*>(dst) = v;
}

namespace {

constexpr size_t WS_ALIGN = 256;
size_t align_up(size_t n) { return (n + WS_ALIGN - 1) / WS_ALIGN * WS_ALIGN; }

// Workspace of one call: fixed buffers, then one partial area reused by
// every chunk launch (they run in stream order).
struct FastLayout {
    bool multi;                    // the staged multi-partition launch serves the call
    size_t lse_n;                  // [B, H, Q] f32
    std::vector<size_t> q_low, kc, vc, kb, vb, out_l, lse_l;  // per group
    size_t partials;
    size_t total;
};

// Batch items that have their own center table (0: one shared table).
int table_batches(const nkv_codec& c, int B) {
    if (c.n_segments > 0) return c.segments[0].centers_batch_stride ? B : 1;
    return c.centers_batch_stride ? B : 1;
}

bool has_centers(const nkv_codec& c) {
    return c.n_segments > 0 ? c.segments[0].centers != nullptr : c.centers != nullptr;
}

// Rows of the (concatenated) center table of a codec.
int64_t table_rows(const nkv_codec& c) {
    if (c.n_segments == 0) return c.num_centers;
    const nkv_segment& last = c.segments[c.n_segments - 1];
    return last.center_base + last.num_centers;
}

// The queries the reader groups project: the pre-RoPE / pre-camera queries
// when given, else attend.q.
bool reader_q_pre(const nkv_fast_args* f) { return f->q_pre != nullptr; }

int validate(const nkv_fast_args* f) {
    NKV_REQUIRE(f, NKV_ERR_INVALID, "null args");
    const nkv_attend_args& a = f->attend;
    NKV_REQUIRE(a.B >= 1 && a.H >= 1 && a.D == 128, NKV_ERR_UNSUPPORTED,
                "fast attend supports D == 128");
    NKV_REQUIRE(a.Q >= 0 && a.N >= 0 && a.Nc >= 0, NKV_ERR_INVALID, "negative length");
    NKV_REQUIRE(!a.hist_rows, NKV_ERR_INVALID,
                "fast attend selects history rows with protect_rows / low_rows");
    const bool readers = f->n_low > 0 && f->num_groups > 0;
    if (a.N > 0) {
        int rc = check_segments(a.key, a.N);
        if (rc) return rc;
        rc = check_segments(a.value, a.N);
        if (rc) return rc;
        if (readers)
            for (const nkv_codec* c : {&a.key, &a.value})
                if (c->n_segments > 0 && has_centers(*c))
                    for (int i = 1; i < c->n_segments; ++i)
                        NKV_REQUIRE((c->segments[i].centers_batch_stride != 0) ==
                                        (c->segments[0].centers_batch_stride != 0),
                                    NKV_ERR_UNSUPPORTED,
                                    "reader groups need segments that all share or all have "
                                    "per-batch center tables");
    }
    if (readers && a.rope)
        NKV_REQUIRE(f->q_pre && f->q_rope, NKV_ERR_INVALID,
                    "RoPE of the reader groups needs q_pre and q_rope");
    if (readers && a.camera)
        NKV_REQUIRE(f->q_pre && f->q_camera, NKV_ERR_INVALID,
                    "the camera of the reader groups needs q_pre and q_camera");
    if (f->q_pre)
        NKV_REQUIRE(reinterpret_cast<uintptr_t>(f->q_pre) % 16 == 0 && f->qp_sb % 8 == 0 &&
                        f->qp_st % 8 == 0 && f->qp_sh % 8 == 0,
                    NKV_ERR_INVALID, "q_pre must be 16-byte aligned with strides divisible by 8");
    if (a.rope) {
        RopeDev chk;
        int rc = rope_from_abi(a.rope, a.D, &chk);
        if (rc) return rc;
        NKV_REQUIRE(a.N <= rope_rows_covered(a.rope),
                    NKV_ERR_INVALID, "more history tokens than the RoPE frames cover");
        if (readers) {
            NKV_REQUIRE(f->q_rope, NKV_ERR_INVALID, "RoPE of the reader groups needs q_rope");
            rc = rope_from_abi(f->q_rope, a.D, &chk);
            if (rc) return rc;
            NKV_REQUIRE(a.Q <= rope_rows_covered(f->q_rope),
                        NKV_ERR_INVALID, "more queries than the query RoPE frames cover");
        }
    }
    if (a.camera) {
        CameraDev chk;
        int rc = camera_from_abi(a.camera, a.D, a.B, &chk);
        if (rc) return rc;
        NKV_REQUIRE(a.camera->layout == NKV_CAMERA_FULL, NKV_ERR_UNSUPPORTED,
                    "fast attend's camera supports the FULL layout (CN/mg35.py:131-132)");
        if (readers) {
            NKV_REQUIRE(f->q_camera, NKV_ERR_INVALID,
                        "the camera of the reader groups needs q_camera (P^T of the queries)");
            rc = camera_from_abi(f->q_camera, a.D, a.B, &chk);
            if (rc) return rc;
        }
    }
    if (f->o_camera) {
        CameraDev chk;
        int rc = camera_from_abi(f->o_camera, a.D, a.B, &chk);
        if (rc) return rc;
        NKV_REQUIRE(f->o_camera->layout == NKV_CAMERA_FULL, NKV_ERR_UNSUPPORTED,
                    "o_camera supports the FULL layout (CN/mg35.py:131-132)");
    }
    NKV_REQUIRE(f->n_protect >= 0 && f->n_low >= 0 && f->n_protect <= a.N && f->n_low <= a.N,
                NKV_ERR_INVALID, "protected/low row counts out of range");
    NKV_REQUIRE(f->n_protect == 0 || f->protect_rows, NKV_ERR_INVALID, "protect_rows missing");
    NKV_REQUIRE(f->n_low == 0 || f->low_rows, NKV_ERR_INVALID, "low_rows missing");
    NKV_REQUIRE(f->num_groups >= 0 && (f->num_groups == 0 || f->groups), NKV_ERR_INVALID,
                "groups missing");
    if (a.Q > 0) NKV_REQUIRE(a.q && a.out, NKV_ERR_INVALID, "q and out required");
    if (a.Q > 0)
        NKV_REQUIRE(rows16(a.q, a.q_sb, a.q_st, a.q_sh) && rows16(a.out, a.o_sb, a.o_st, a.o_sh),
                    NKV_ERR_INVALID, "q and out must be 16-byte aligned with strides divisible by 8");
    if (a.Nc > 0)
        NKV_REQUIRE(rows16(a.k_cur, a.k_sb, a.k_st, a.k_sh) &&
                        rows16(a.v_cur, a.v_sb, a.v_st, a.v_sh),
                    NKV_ERR_INVALID,
                    "k_cur and v_cur must be 16-byte aligned with strides divisible by 8");
    if (a.Nc > 0) NKV_REQUIRE(a.k_cur && a.v_cur, NKV_ERR_INVALID, "current K/V missing");
    NKV_REQUIRE(!a.cur_mask || (a.n_groups >= 1 && a.cur_mask_words >= cdiv(a.Nc, 32)),
                NKV_ERR_INVALID, "the current-key mask needs n_groups >= 1 and "
                "cur_mask_words >= ceil(Nc / 32)");
    if (f->n_low > 0 || f->n_protect > 0)
        NKV_REQUIRE((a.key.packed || a.key.n_segments > 0) &&
                        (a.value.packed || a.value.n_segments > 0),
                    NKV_ERR_INVALID, "history codecs missing");
    for (int g = 0; g < f->num_groups; ++g) {
        const nkv_reader_group& G = f->groups[g];
        NKV_REQUIRE(G.num_heads >= 1 && G.num_heads <= a.H && G.heads, NKV_ERR_INVALID,
                    "reader group needs 1..H heads");
        NKV_REQUIRE(G.d == 32 || G.d == 64 || G.d == 128, NKV_ERR_UNSUPPORTED,
                    "reader width d must be 32, 64 or 128");
        NKV_REQUIRE(G.q_reduce || G.d == a.D, NKV_ERR_INVALID, "identity q_reduce needs d == D");
        NKV_REQUIRE(G.k_affine || G.d == a.D, NKV_ERR_INVALID, "identity k_affine needs d == D");
        NKV_REQUIRE(G.k_read && G.v_read, NKV_ERR_INVALID, "reader group needs k_read and v_read");
        NKV_REQUIRE(!a.rope || G.rope_pairs || G.d == a.D, NKV_ERR_INVALID,
                    "RoPE of a reader group narrower than D needs rope_pairs");
        NKV_REQUIRE(!a.camera || G.cam_blocks || G.d == a.D, NKV_ERR_INVALID,
                    "the camera of a reader group narrower than D needs cam_blocks");
    }
    return NKV_OK;
}

ChunkLaunchDesc native_desc(const nkv_fast_args* f, float* lse_n) {
    const nkv_attend_args& a = f->attend;
    ChunkLaunchDesc d{};
    d.B = a.B;
    d.H = a.H;
    d.dk = a.D;
    d.Q = a.Q;
    d.N = a.N;
    d.n_rows = f->n_protect;
    d.rows = f->protect_rows;
    d.Nc = a.Nc;
    d.softmax_scale = a.softmax_scale;
    d.q = a.q;
    d.q_sb = a.q_sb;
    d.q_st = a.q_st;
    d.q_sh = a.q_sh;
    d.k_cur = a.k_cur;
    d.k_sb = a.k_sb;
    d.k_st = a.k_st;
    d.k_sh = a.k_sh;
    d.v_cur = a.v_cur;
    d.v_sb = a.v_sb;
    d.v_st = a.v_st;
    d.v_sh = a.v_sh;
    const int HD = a.H * a.D;
    d.key = chunk_codec_from(a.key, a.D, HD);
    d.value = chunk_codec_from(a.value, a.D, HD);
    d.out = a.out;
    d.o_sb = a.o_sb;
    d.o_st = a.o_st;
    d.o_sh = a.o_sh;
    d.lse = lse_n;
    d.ev_begin = a.ev_kernel_begin;
    d.ev_end = a.ev_kernel_end;
    d.cur_mask = a.cur_mask;
    d.q_group = a.q_group;
    d.n_groups = a.n_groups;
    d.mask_words = a.cur_mask_words;
    return d;
}

// Identity readers (k_affine / v_affine null): their center tables and
// means are the layer's own (bf16 columns of head heads[i]; the mean applied
// as bf16), read through the head map instead of projected copies.
// Identity q_reduce: the queries are the layer's (pre-RoPE when given).
// The staged multi-partition launch reads them so; the per-group launches
// take projected copies.
struct ReaderIdent {
    bool q, k, v;
};

// With read-time RoPE the reader queries are always formed from q_pre and
// rotated at the query positions, as the per-group path does.
ReaderIdent reader_ident(const nkv_fast_args* f, const nkv_reader_group& G, bool multi) {
    return multi ? ReaderIdent{!G.q_reduce && !f->attend.rope && !f->attend.camera, !G.k_affine,
                               !G.v_affine}
                 : ReaderIdent{false, false, false};
}

// Low-partition launch of group g over the workspace tables.
ChunkLaunchDesc low_desc(const nkv_fast_args* f, int g, unsigned char* ws, const FastLayout& L,
                         bool multi = false) {
    const ReaderIdent id = reader_ident(f, f->groups[g], multi);
    const nkv_attend_args& a = f->attend;
    const nkv_reader_group& G = f->groups[g];
    const int nh = G.num_heads, dd = G.d, D = a.D;
    ChunkLaunchDesc d{};
    d.B = a.B;
    d.H = nh;
    d.dk = dd;
    d.Q = a.Q;
    d.N = a.N;
    d.n_rows = f->n_low;
    d.rows = f->low_rows;
    d.Nc = 0;
    d.softmax_scale = a.softmax_scale;
    auto at = [&](size_t off) { return ws ? ws + off : nullptr; };
    if (id.q) {
        // the layer's queries of heads G.heads
        const bool pre = reader_q_pre(f);
        d.q = reinterpret_cast<const uint16_t*>(pre ? f->q_pre : a.q);
        d.q_sb = pre ? f->qp_sb : a.q_sb;
        d.q_st = pre ? f->qp_st : a.q_st;
        d.q_sh = pre ? f->qp_sh : a.q_sh;
        d.q_heads = G.heads;
        d.q_heads_n = a.H;
    } else {
        d.q = reinterpret_cast<const uint16_t*>(at(L.q_low[g]));  // [B, Q, nh, d]
        d.q_sb = a.Q * nh * dd;
        d.q_st = (int64_t)nh * dd;
        d.q_sh = dd;
    }
    for (int cc = 0; cc < 2; ++cc) {
        const nkv_codec& c = cc ? a.value : a.key;
        ChunkCodec v{};
        v.r = c.r;
        v.group = c.group;
        v.scale_dtype = c.scale_dtype;
        if (c.n_segments > 0) {
            v.seg = c.segments_dev;
            v.n_seg = c.n_segments;
            v.seg_flat = 1;
        } else {
            v.packed = c.packed;
            v.scales = c.scales;
            v.ids = c.centers ? c.ids : nullptr;
            v.id_bytes = c.id_bytes;
            v.num_centers = c.num_centers;
        }
        const int width = cc ? D : dd;
        v.w = cc ? G.v_read : G.k_read;
        v.w_hs = (int64_t)width * c.r;
        if (cc ? id.v : id.k) {
            // the layer's tables, as the native partition reads them
            const ChunkCodec own = chunk_codec_from(c, D, a.H * D);
            v.seg_flat = own.seg_flat;
            v.has_centers = own.has_centers;
            v.centers = own.centers;
            v.c_bs = own.c_bs;
            v.c_rs = own.c_rs;
            v.c_hs = own.c_hs;
            v.bias = own.bias;
            v.bias_hs = own.bias_hs;
            v.c_heads = G.heads;
            v.c_heads_n = a.H;
            (cc ? d.value : d.key) = v;
            continue;
        }
        if (has_centers(c)) {
            // projected table [tables][nh][C][width]
            const int64_t C = table_rows(c);
            v.has_centers = 1;
            v.centers = reinterpret_cast<const uint16_t*>(at(cc ? L.vc[g] : L.kc[g]));
            v.c_rs = width;
            v.c_hs = C * width;
            v.c_bs = table_batches(c, a.B) > 1 ? (int64_t)nh * C * width : 0;
        }
        if (c.mean) {
            v.bias = reinterpret_cast<const float*>(at(cc ? L.vb[g] : L.kb[g]));
            v.bias_hs = width;
        }
        (cc ? d.value : d.key) = v;
    }
    d.out = reinterpret_cast<uint16_t*>(at(L.out_l[g]));  // [B, Q, nh, D]
    d.o_sb = a.Q * nh * D;
    d.o_st = (int64_t)nh * D;
    d.o_sh = D;
    d.lse = reinterpret_cast<float*>(at(L.lse_l[g]));
    return d;
}

// A partition's read-time transforms as the launches apply them: the
// history keys' RoPE at their codec rows (a reader group's keys on its pair
// map) and the camera's P^-1 (a reader group's keys on its block map).  The
// workspace plan depends on them, so the size query applies them too.
void add_transforms(const nkv_fast_args* f, const nkv_reader_group* G, ChunkLaunchDesc& d) {
    const nkv_attend_args& a = f->attend;
    if (a.rope) {
        rope_from_abi(a.rope, a.D, &d.rope);
        if (G) d.rope.pairs = G->rope_pairs;
    }
    if (a.camera) {
        camera_from_abi(a.camera, a.D, a.B, &d.cam);
        if (G) d.cam.blocks = G->cam_blocks;
    }
}

// The partitions of the staged multi-partition launch: the native one, then
// every reader group (heads[1 + g] = its heads).  With read-time RoPE every
// partition rotates its history keys at their codec rows, a reader group on
// its pair map; with the camera every partition's history rows take P^-1, a
// reader group's keys on its block map.
int multi_descs(const nkv_fast_args* f, unsigned char* ws, const FastLayout& L,
                ChunkLaunchDesc* d, const int32_t** heads) {
    d[0] = native_desc(f, f->attend.lse);
    add_transforms(f, nullptr, d[0]);
    heads[0] = nullptr;
    for (int g = 0; g < f->num_groups; ++g) {
        d[1 + g] = low_desc(f, g, ws, L, true);
        add_transforms(f, &f->groups[g], d[1 + g]);
        heads[1 + g] = f->groups[g].heads;
    }
    return 1 + f->num_groups;
}

// One decode, one flash and one combine launch (and with the camera one
// tile pass) serve the whole call (every partition merged in the combine,
// no per-group merge) when the native partition and the reader groups fit
// one staged launch.
bool use_multi(const nkv_fast_args* f) {
    if (f->n_low == 0 || f->num_groups < 1 || f->num_groups + 1 > NKV_MAX_PARTS)
        return false;
    FastLayout L{};
    for (auto* v : {&L.q_low, &L.kc, &L.vc, &L.kb, &L.vb, &L.out_l, &L.lse_l})
        v->assign(f->num_groups, 0);
    ChunkLaunchDesc d[NKV_MAX_PARTS];
    const int32_t* heads[NKV_MAX_PARTS];
    const int n = multi_descs(f, nullptr, L, d, heads);
    return staged_multi_supported(d, n);
}

FastLayout layout(const nkv_fast_args* f) {
    const nkv_attend_args& a = f->attend;
    FastLayout L;
    L.multi = use_multi(f);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align_up(bytes);
        return o;
    };
    L.lse_n = take(a.lse || L.multi ? 0 : (size_t)a.B * a.H * a.Q * sizeof(float));
    for (int g = 0; g < f->num_groups; ++g) {
        const nkv_reader_group& G = f->groups[g];
        const ReaderIdent id = reader_ident(f, G, L.multi);
        const size_t nh = G.num_heads, dd = G.d, D = a.D;
        L.q_low.push_back(take(id.q ? 0 : (size_t)a.B * a.Q * nh * dd * 2));
        const size_t kt = has_centers(a.key) && !id.k ? (size_t)table_batches(a.key, a.B) : 0;
        const size_t vt = has_centers(a.value) && !id.v ? (size_t)table_batches(a.value, a.B) : 0;
        L.kc.push_back(take(kt * nh * (size_t)table_rows(a.key) * dd * 2));
        L.vc.push_back(take(vt * nh * (size_t)table_rows(a.value) * D * 2));
        L.kb.push_back(take(id.k ? 0 : nh * dd * sizeof(float)));
        L.vb.push_back(take(id.v ? 0 : nh * D * sizeof(float)));
        L.out_l.push_back(take(L.multi ? 0 : (size_t)a.B * a.Q * nh * D * 2));
        L.lse_l.push_back(take(L.multi ? 0 : (size_t)a.B * nh * a.Q * sizeof(float)));
    }
    size_t part;
    if (L.multi) {
        ChunkLaunchDesc d[NKV_MAX_PARTS];
        const int32_t* heads[NKV_MAX_PARTS];
        const int n = multi_descs(f, nullptr, L, d, heads);
        part = staged_multi_workspace(d, n);
    } else {
        ChunkLaunchDesc nd = native_desc(f, nullptr);
        add_transforms(f, nullptr, nd);
        part = chunk_launch_workspace(nd);
        for (int g = 0; g < f->num_groups; ++g) {
            ChunkLaunchDesc ld = low_desc(f, g, nullptr, L);
            add_transforms(f, &f->groups[g], ld);
            part = std::max(part, chunk_launch_workspace(ld));
        }
    }
    L.partials = take(part);
    L.total = off;
    return L;
}

template <bool XF, bool OF>
int project(hipStream_t s, const void* x, int64_t x_b, int64_t x_m, int64_t x_h,
            const nkv_segment* seg, int n_seg, const int32_t* heads, int H, const uint16_t* w,
            int D, int E, int nb, int nh, int64_t M, void* out, int64_t o_b, int64_t o_i,
            int64_t o_m) {
    const int64_t total = (int64_t)nb * nh * M * E;
    if (total == 0) return NKV_OK;
    // 16-byte operand loads need aligned rows (8 bf16 or 4 fp32 elements);
    // segment tables are [*, C, HD] bf16 tensors (HD a multiple of 8)
    const int64_t el = XF ? 4 : 8;
    const bool aligned = seg ? x_m % el == 0 && x_h % el == 0
                             : reinterpret_cast<uintptr_t>(x) % 16 == 0 && x_b % el == 0 &&
                                   x_m % el == 0 && x_h % el == 0;
    if (w && aligned && D <= PJ_MAXD && D % 16 == 0 && E % 32 == 0 && E <= PJ_MAXE) {
        project_mfma_kernel<XF, OF><<<dim3((unsigned)cdiv(M, PJ_ROWS), (unsigned)nh, (unsigned)nb),
                                      256, 0, s>>>(x, x_b, x_m, x_h, seg, n_seg, heads, H, w, D, E,
                                                   M, out, o_b, o_i, o_m);
    } else {
        project_kernel<XF, OF><<<dim3((unsigned)cdiv(total, 256)), 256, 0, s>>>(
            x, x_b, x_m, x_h, seg, n_seg, heads, H, w, D, E, nb, nh, M, out, o_b, o_i, o_m);
    }
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

// The tables reader group g reads through (CN/core.py:155-204): q_low, and
// its projected center tables and means, for the parts that are not the
// layer's own (identity readers of the multi-partition launch).
int reader_tables(hipStream_t s, const nkv_fast_args* f, int g, unsigned char* ws,
                  const FastLayout& L, const RopeDev& qrope, const CameraDev& qcam) {
    const nkv_attend_args& a = f->attend;
    const nkv_reader_group& G = f->groups[g];
    const ReaderIdent id = reader_ident(f, G, L.multi);
    const int D = a.D, HD = a.H * a.D;
    const int nh = G.num_heads, dd = G.d;
    int rc = NKV_OK;
    // q_low [B, Q, nh, d] from the pre-RoPE, pre-camera queries when
    // given, then rotated / transformed on its retained pairs and blocks by
    // query_transforms (an identity q_reduce takes them through the head map
    // in that pass)
    uint16_t* q_low = reinterpret_cast<uint16_t*>(ws + L.q_low[g]);
    const bool pre = reader_q_pre(f);
    const uint16_t* qsrc = reinterpret_cast<const uint16_t*>(pre ? f->q_pre : a.q);
    const int64_t qs_b = pre ? f->qp_sb : a.q_sb, qs_t = pre ? f->qp_st : a.q_st,
                  qs_h = pre ? f->qp_sh : a.q_sh;
    const bool xform = a.rope || a.camera;
    if (!id.q && (G.q_reduce || !xform)) {
        rc = project<false, false>(s, qsrc, qs_b, qs_t, qs_h, nullptr, 0, G.heads, a.H,
                                   G.q_reduce, D, dd, a.B, nh, a.Q, q_low, a.Q * nh * dd, dd,
                                   (int64_t)nh * dd);
        if (rc) return rc;
    }
    for (int cc = 0; cc < 2 && f->n_low > 0; ++cc) {
        if (cc ? id.v : id.k) continue;
        const nkv_codec& c = cc ? a.value : a.key;
        const int width = cc ? D : dd;
        const uint16_t* aff = cc ? G.v_affine : G.k_affine;
        if (has_centers(c)) {
            // [tables][nh][C][width] = center columns of each head . affine
            const int nb = table_batches(c, a.B);
            const int64_t C = table_rows(c);
            rc = project<false, false>(
                s, c.centers, c.centers_batch_stride, HD, D,
                c.n_segments > 0 ? c.segments_dev : nullptr, c.n_segments, G.heads, a.H, aff,
                D, width, nb, nh, C, ws + (cc ? L.vc[g] : L.kc[g]), (int64_t)nh * C * width,
                C * width, width);
            if (rc) return rc;
        }
        if (c.mean) {
            // [nh][width] = bf16(mean of each head) . affine
            rc = project<true, true>(s, c.mean, 0, 0, D, nullptr, 0, G.heads, a.H, aff, D,
                                     width, 1, nh, 1, ws + (cc ? L.vb[g] : L.kb[g]), 0, width,
                                     0);
            if (rc) return rc;
        }
    }
    return NKV_OK;
}

// The reader queries' RoPE and camera for every group that needs them, in
// launches of up to QL_MAX groups (after reader_tables has projected them).
int query_transforms(hipStream_t s, const nkv_fast_args* f, unsigned char* ws,
                     const FastLayout& L, const RopeDev& qrope, const CameraDev& qcam) {
    const nkv_attend_args& a = f->attend;
    if (!a.rope && !a.camera) return NKV_OK;
    const bool pre = reader_q_pre(f);
    QueryLowBatch P{};
    P.H = a.H;
    P.B = a.B;
    P.Q = a.Q;
    P.s_b = pre ? f->qp_sb : a.q_sb;
    P.s_t = pre ? f->qp_st : a.q_st;
    P.s_h = pre ? f->qp_sh : a.q_sh;
    if (a.rope) P.pos = qrope;
    if (a.camera) P.cam = qcam;
    auto flush = [&]() -> int {
        if (P.n == 0) return NKV_OK;
        query_low_kernel<<<dim3((unsigned)cdiv(P.first[P.n], 256)), 256, 0, s>>>(P);
        NKV_LAUNCH_CHECK();
        P.n = 0;
        return NKV_OK;
    };
    for (int g = 0; g < f->num_groups; ++g) {
        const nkv_reader_group& G = f->groups[g];
        if (reader_ident(f, G, L.multi).q) continue;
        QueryLowGroup& q = P.g[P.n];
        q.q_low = reinterpret_cast<uint16_t*>(ws + L.q_low[g]);
        q.src = G.q_reduce ? nullptr : reinterpret_cast<const uint16_t*>(pre ? f->q_pre : a.q);
        q.heads = G.heads;
        q.pairs = a.rope ? G.rope_pairs : nullptr;
        q.cams = a.camera ? G.cam_blocks : nullptr;
        q.nh = G.num_heads;
        q.d = G.d;
        q.ostride = G.d;
        P.first[P.n + 1] = P.first[P.n] + (int64_t)a.B * a.Q * G.num_heads * (G.d / 8);
        if (++P.n == QL_MAX) {
            int rc = flush();
            if (rc) return rc;
        }
    }
    return flush();
}

}  // namespace

}  // namespace nkv

using namespace nkv;

extern "C" size_t nkv_fast_attend_workspace_size(const nkv_fast_args* f) {
    clear_error();
    if (validate(f)) return 0;
    return layout(f).total;
}

extern "C" int nkv_fast_attend(void* stream, const nkv_fast_args* f, void* workspace,
                               size_t workspace_bytes) {
    clear_error();
    int rc = validate(f);
    if (rc) return rc;
    const nkv_attend_args& a = f->attend;
    if (a.Q == 0) return NKV_OK;
    hipStream_t s = (hipStream_t)stream;
    const FastLayout L = layout(f);
    NKV_REQUIRE(workspace && workspace_bytes >= L.total, NKV_ERR_WORKSPACE,
                "workspace missing or smaller than nkv_fast_attend_workspace_size()");
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    const size_t part_bytes = L.total - L.partials;
    // the native partition's LSE goes to the caller's lse when it asked for
    // one; the merges then update it in place
    float* lse_n = a.lse ? a.lse : reinterpret_cast<float*>(ws + L.lse_n);

    // the reader queries' positions and camera (the history's are added to
    // each partition's launch by add_transforms)
    RopeDev qrope{};
    if (a.rope && f->q_rope) rope_from_abi(f->q_rope, a.D, &qrope);
    CameraDev qcam{};
    if (a.camera && f->q_camera) camera_from_abi(f->q_camera, a.D, a.B, &qcam);

    if (L.multi) {
        // the reader tables, then every partition in one staged launch whose
        // combine merges each head's partitions into out / lse
        for (int g = 0; g < f->num_groups; ++g) {
            rc = reader_tables(s, f, g, ws, L, qrope, qcam);
            if (rc) return rc;
        }
        rc = query_transforms(s, f, ws, L, qrope, qcam);
        if (rc) return rc;
        ChunkLaunchDesc d[NKV_MAX_PARTS];
        const int32_t* heads[NKV_MAX_PARTS];
        const int n = multi_descs(f, ws, L, d, heads);
        CameraDev ocam{};
        if (f->o_camera) camera_from_abi(f->o_camera, a.D, a.B, &ocam);
        return staged_multi_launch(s, d, n, heads, f->low_shift, f->ls_sb, f->ls_sh,
                                   ws + L.partials, part_bytes, ocam);
    }

    // P of the query rows on the merged output, when the call applies it
    auto finish = [&]() -> int {
        if (!f->o_camera) return NKV_OK;
        CameraDev ocam{};
        camera_from_abi(f->o_camera, a.D, a.B, &ocam);
        return camera_apply_inplace(s, ocam, a.B, a.Q, a.H, a.D, a.out, a.o_sb, a.o_st, a.o_sh);
    };

    // 1. native partition -> out, lse_n
    ChunkLaunchDesc nd = native_desc(f, lse_n);
    add_transforms(f, nullptr, nd);
    rc = chunk_launch(s, nd, ws + L.partials, part_bytes);
    if (rc) return rc;
    // no low rows: the native partition is the whole attention
    if (f->n_low == 0) return finish();

    // 2-3. reader groups: every group's tables and queries, then each
    // group's launch and merge
    for (int g = 0; g < f->num_groups; ++g) {
        rc = reader_tables(s, f, g, ws, L, qrope, qcam);
        if (rc) return rc;
    }
    rc = query_transforms(s, f, ws, L, qrope, qcam);
    if (rc) return rc;
    for (int g = 0; g < f->num_groups; ++g) {
        const nkv_reader_group& G = f->groups[g];
        const int nh = G.num_heads, D = a.D;
        ChunkLaunchDesc ld = low_desc(f, g, ws, L);
        add_transforms(f, &G, ld);
        rc = chunk_launch(s, ld, ws + L.partials, part_bytes);
        if (rc) return rc;
        const int64_t threads = (int64_t)a.B * a.Q * nh * (D / 8);
        group_merge_kernel<<<dim3((unsigned)cdiv(threads, 256)), 256, 0, s>>>(
            a.B, a.Q, nh, D, G.heads, a.out, a.o_sb, a.o_st, a.o_sh, lse_n, a.H,
            reinterpret_cast<const uint16_t*>(ws + L.out_l[g]),
            reinterpret_cast<const float*>(ws + L.lse_l[g]), a.lse, f->low_shift, f->ls_sb,
            f->ls_sh);
        NKV_LAUNCH_CHECK();
    }
    return finish();
}

extern "C" int nkv_reader_rows(void* stream, const nkv_reader_rows_args* a) {
    clear_error();
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null args");
    NKV_REQUIRE(a->B >= 1 && a->H >= 1 && a->nh >= 1 && a->S >= 0, NKV_ERR_INVALID,
                "B, H and nh must be >= 1 and S >= 0");
    NKV_REQUIRE(a->D > 0 && a->D % 8 == 0 && a->D <= 512, NKV_ERR_INVALID,
                "D must be a positive multiple of 8 (at most 512)");
    NKV_REQUIRE(a->E > 0 && a->E % 8 == 0 && a->out_width >= a->E && a->out_width % 8 == 0,
                NKV_ERR_INVALID, "E and out_width must be multiples of 8 with E <= out_width");
    NKV_REQUIRE(a->w || a->E == a->D, NKV_ERR_INVALID, "without w the rows keep their width (E == D)");
    if (a->S == 0) return NKV_OK;
    NKV_REQUIRE(a->x && a->heads && a->out, NKV_ERR_INVALID, "x, heads and out are required");
    NKV_REQUIRE(rows16(a->x, a->x_sb, a->x_st, a->x_sh) &&
                    reinterpret_cast<uintptr_t>(a->out) % 16 == 0,
                NKV_ERR_INVALID, "x rows and out must be 16-byte aligned (strides divisible by 8)");
    hipStream_t s = (hipStream_t)stream;
    QueryLowBatch P{};
    P.H = a->H;
    P.B = a->B;
    P.Q = a->S;
    P.s_b = a->x_sb;
    P.s_t = a->x_st;
    P.s_h = a->x_sh;
    if (a->rope) {
        int rc = rope_from_abi(a->rope, a->D, &P.pos);
        if (rc) return rc;
    }
    if (a->camera) {
        NKV_REQUIRE(a->camera->layout == NKV_CAMERA_FULL, NKV_ERR_UNSUPPORTED,
                    "reader rows take the camera on their 8-dim blocks (the FULL layout)");
        int rc = camera_from_abi(a->camera, a->D, a->B, &P.cam);
        if (rc) return rc;
    }
    if (a->w) {
        // y = bf16(x[b, s, heads[i]] . w[i]) into out [B, S, nh, out_width]
        const int64_t W = a->out_width;
        int rc = project<false, false>(s, a->x, a->x_sb, a->x_st, a->x_sh, nullptr, 0, a->heads, a->H,
                                       a->w, a->D, a->E, a->B, a->nh, a->S, a->out,
                                       a->S * a->nh * W, W, a->nh * W);
        if (rc) return rc;
        if (!a->rope && !a->camera && a->out_width == a->E) return NKV_OK;
    }
    // RoPE, camera, the identity copy through the head map and the zero columns
    QueryLowGroup& g = P.g[0];
    g.q_low = a->out;
    g.src = a->w ? nullptr : a->x;
    g.heads = a->heads;
    g.pairs = a->rope ? a->pairs : nullptr;
    g.cams = a->camera ? a->blocks : nullptr;
    g.nh = a->nh;
    g.d = a->E;
    g.ostride = a->out_width;
    P.n = 1;
    P.first[1] = (int64_t)a->B * a->S * a->nh * (a->out_width / 8);
    query_low_kernel<<<dim3((unsigned)cdiv(P.first[1], 256)), 256, 0, s>>>(P);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
