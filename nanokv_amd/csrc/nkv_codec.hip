// nkv_codec.hip -- NanoKV chunk codec on gfx950: INT4 quantise/pack, unpack,
// nearest-center assignment, encoder projection and full-width decode.
//
// This translation unit is compiled with -ffp-contract=off: the quantiser and
// the decode epilogue are bit-exact restatements whose rounding points must
// not be fused away.
#include "nkv_common.h"

namespace nkv {

// ============================================================ quantiser
// One thread per (row, group).  Each thread reads its group with 16-byte
// loads, computes the exact amax (order-free), the IEEE-divided scale, and
// writes group/2 packed bytes plus one scale.  Reference: MG:349-351 (fp32
// arithmetic as in HY kv_codecs.py:244-255; bf16 arithmetic as MG deploys
// it) and _pack_int4 MG:282-292.
template <int QUANT_MODE>
__device__ __forceinline__ void quant_pack_group(const float* __restrict__ coeff, int64_t rows,
                                                 int r, int group, int scale_dtype,
                                                 uint8_t* __restrict__ packed,
                                                 uint16_t* __restrict__ scales, int64_t gid) {
    const int ngroups = r / group;
    if (gid >= rows * ngroups) return;
    const int64_t row = gid / ngroups;
    const int g = (int)(gid - row * ngroups);
    const float* x = coeff + row * r + (int64_t)g * group;

    float amax = 0.0f;
    for (int j = 0; j < group; j += 4) {
        f32x4 v = *reinterpret_cast<const f32x4*>(x + j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float a = QUANT_MODE == NKV_QUANT_BF16 ? bf16_round(v[e]) : v[e];
            a = fabsf(a);
            amax = (a > amax || a != a) ? a : amax;  // NaN propagates like torch.amax
        }
    }
    float s;
    const float eps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps
    float clamped = (amax > eps || amax != amax) ? amax : eps;
    if (QUANT_MODE == NKV_QUANT_BF16) {
        s = bf16_round(__fdiv_rn(bf16_round(clamped), 7.0f));
    } else {
        s = __fdiv_rn(clamped, 7.0f);
    }
    scales[row * ngroups + g] =
        scale_dtype == NKV_DTYPE_FP16 ? f32_to_f16_bits(s) : f32_to_bf16_bits(s);

    uint8_t* out = packed + row * (r / 2) + (int64_t)g * (group / 2);
    for (int j = 0; j < group; j += 8) {
        f32x4 v0 = *reinterpret_cast<const f32x4*>(x + j);
        f32x4 v1 = *reinterpret_cast<const f32x4*>(x + j + 4);
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = e < 4 ? v0[e] : v1[e - 4];
            if (QUANT_MODE == NKV_QUANT_BF16) v = bf16_round(v);
            float q = __fdiv_rn(v, s);
            if (QUANT_MODE == NKV_QUANT_BF16) q = bf16_round(q);
            float rq = rintf(q);  // round half to even, as torch.round
            int c = rq != rq ? 0 : (int)fminf(fmaxf(rq, -7.0f), 7.0f);
            word |= (uint32_t)(c + 7) << (4 * e);
        }
        *reinterpret_cast<uint32_t*>(out + j / 2) = word;
    }
}

template <int QUANT_MODE>
__global__ void __launch_bounds__(256) quant_pack_kernel(const float* __restrict__ coeff,
                                                         int64_t rows, int r, int group,
                                                         int scale_dtype,
                                                         uint8_t* __restrict__ packed,
                                                         uint16_t* __restrict__ scales) {
    quant_pack_group<QUANT_MODE>(coeff, rows, r, group, scale_dtype, packed, scales,
                                 (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// ============================================================ unpack
// One thread per 8 consecutive codes (4 packed bytes) of one row.
__global__ void __launch_bounds__(256) unpack_kernel(const uint8_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ scales,
                                                     int scale_dtype,
                                                     const int32_t* __restrict__ row_index,
                                                     int64_t rows, int r, int group,
                                                     uint16_t* __restrict__ out) {
    const int per_row = r / 8;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= rows * per_row) return;
    const int64_t i = tid / per_row;
    const int j0 = (int)(tid - i * per_row) * 8;
    const int64_t src = row_index ? (int64_t)row_index[i] : i;
    const uint32_t word = *reinterpret_cast<const uint32_t*>(packed + src * (r / 2) + j0 / 2);
    const float s = scale_bits_to_f32(scales[src * (r / group) + j0 / group], scale_dtype);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float lo = (float)((int)((word >> (8 * e)) & 15u) - 7) * s;
        float hi = (float)((int)((word >> (8 * e + 4)) & 15u) - 7) * s;
        o[e] = pack_bf16x2(lo, hi);
    }
    *reinterpret_cast<u32x4*>(out + i * r + j0) = o;
}

// ============================================================ assignment
// fp64 nearest-center search.  A 256-thread block owns 32 rows and walks the
// center table in chunks of 64; each thread keeps a 2-row x 4-center fp64
// register tile.  Per chunk the block stages x[32 x 64] (fp32) and
// c[64 x 64] (bf16) in LDS along HD.  ||c||^2 is accumulated by the same
// threads (only the thread column that owns row 0 keeps it).  Distances are
// ||c||^2 - 2 x.c (||x||^2 is constant per row); ties keep the lowest index.
constexpr int AS_ROWS = 32, AS_CENT = 64, AS_K = 64;

template <int ID_BYTES>
__device__ __forceinline__ void store_id(void* ids, int64_t i, int v) {
    if (ID_BYTES == 1) reinterpret_cast<uint8_t*>(ids)[i] = (uint8_t)v;
    else if (ID_BYTES == 2) reinterpret_cast<uint16_t*>(ids)[i] = (uint16_t)v;
    else reinterpret_cast<int32_t*>(ids)[i] = v;
}

// A center element as fp32: bf16 bits or fp32 (both exact in fp64).
__device__ __forceinline__ float center_value(const uint16_t* c, int64_t i) {
    return bf16_bits_to_f32(c[i]);
}
__device__ __forceinline__ float center_value(const float* c, int64_t i) { return c[i]; }

template <int ID_BYTES, typename CT = uint16_t>
__global__ void __launch_bounds__(256) assign_kernel(const float* __restrict__ x,
                                                     const CT* __restrict__ centers,
                                                     int64_t rows, int C, int HD,
                                                     void* __restrict__ ids) {
    __shared__ float xs[AS_ROWS][AS_K + 1];
    __shared__ float cs[AS_CENT][AS_K + 1];
    __shared__ double red_d[AS_ROWS][16];
    __shared__ int red_c[AS_ROWS][16];

    const int t = threadIdx.x;
    const int tr = t / 16;          // rows tr and tr + 16
    const int tc = t % 16;          // centers tc + 16*j, j = 0..3
    const int64_t row0 = (int64_t)blockIdx.x * AS_ROWS;

    double best[2] = {0.0, 0.0};
    int best_c[2] = {-1, -1};

    for (int c0 = 0; c0 < C; c0 += AS_CENT) {
        double dot[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
        double cc[4] = {0, 0, 0, 0};
        for (int k0 = 0; k0 < HD; k0 += AS_K) {
            __syncthreads();
            // stage x: 32 x 64 fp32 = 2048 values, 8 per thread
            for (int e = t; e < AS_ROWS * AS_K; e += 256) {
                int rr = e / AS_K, kk = e % AS_K;
                int64_t gr = row0 + rr;
                xs[rr][kk] = (gr < rows && k0 + kk < HD) ? x[gr * HD + k0 + kk] : 0.0f;
            }
            for (int e = t; e < AS_CENT * AS_K; e += 256) {
                int cr = e / AS_K, kk = e % AS_K;
                int gc = c0 + cr;
                cs[cr][kk] = (gc < C && k0 + kk < HD)
                                 ? center_value(centers, (int64_t)gc * HD + k0 + kk)
                                 : 0.0f;
            }
            __syncthreads();
            for (int kk = 0; kk < AS_K; ++kk) {
                double xv0 = (double)xs[tr][kk];
                double xv1 = (double)xs[tr + 16][kk];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    double cv = (double)cs[tc + 16 * j][kk];
                    dot[0][j] += xv0 * cv;
                    dot[1][j] += xv1 * cv;
                    cc[j] += cv * cv;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int c = c0 + tc + 16 * j;
            if (c >= C) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                double d = cc[j] - 2.0 * dot[i][j];
                if (best_c[i] < 0 || d < best[i] || (d == best[i] && c < best_c[i])) {
                    best[i] = d;
                    best_c[i] = c;
                }
            }
        }
    }
    // reduce over the 16 center lanes of each row (fixed order: lowest index wins ties)
    red_d[tr][tc] = best[0];
    red_c[tr][tc] = best_c[0];
    red_d[tr + 16][tc] = best[1];
    red_c[tr + 16][tc] = best_c[1];
    __syncthreads();
    if (t < AS_ROWS) {
        double bd = red_d[t][0];
        int bc = red_c[t][0];
        for (int j = 1; j < 16; ++j) {
            int c = red_c[t][j];
            double d = red_d[t][j];
            if (c >= 0 && (bc < 0 || d < bd || (d == bd && c < bc))) {
                bd = d;
                bc = c;
            }
        }
        int64_t gr = row0 + t;
        if (gr < rows) store_id<ID_BYTES>(ids, gr, bc);
    }
}

// fp64 MFMA nearest-center search (v_mfma_f64_16x16x4_f64).  A 256-thread
// block owns 16 rows; wave w takes centers 64*w + [0, 64) of every group of
// 256 as four 16 x 16 output tiles.  Operands come straight from L2: at each
// 16-wide k block lane l supplies x row (l % 16) and center column (l % 16)
// at k = k0 + 4*(l / 16) + [0, 4), one 16-byte x piece and one 8-byte
// center piece per tile for four MFMA steps (any k order is valid for the
// reduction, and A and B use the same one).  Every product of an fp32 x and
// a bf16 center is exact in fp64, so only the order of the fp64 sums differs
// from the fp64 VALU search (relative 1e-16).  ||c||^2 comes from the same
// center pieces.  Output layout: lane l, element e holds row 4e + l/16,
// column l % 16.  Needs HD % 16 == 0, x 16-byte and centers 8-byte aligned.
constexpr int AM_ROWS = 16, AM_AHEAD = 4;
typedef double f64x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool better(double d, int c, double bd, int bc) {
    return bc < 0 || (c >= 0 && (d < bd || (d == bd && c < bc)));
}

// Four consecutive center elements of one lane's k block: 8 bytes of bf16
// or 16 bytes of fp32; element st as an exact fp64.
template <typename CT>
struct CenterPiece;
template <>
struct CenterPiece<uint16_t> {
    using V = u32x2;
    static __device__ __forceinline__ double get(const V& v, int st) {
        const uint32_t w = v[st >> 1];
        return (double)__uint_as_float((st & 1) ? (w & 0xffff0000u) : (w << 16));
    }
};
template <>
struct CenterPiece<float> {
    using V = u32x4;
    static __device__ __forceinline__ double get(const V& v, int st) {
        return (double)__uint_as_float(v[st]);
    }
};

template <int ID_BYTES, typename CT = uint16_t>
__global__ void __launch_bounds__(256) assign_mfma_kernel(const float* __restrict__ x,
                                                          const CT* __restrict__ centers,
                                                          int64_t rows, int C, int HD,
                                                          void* __restrict__ ids) {
    using CP = CenterPiece<CT>;
    __shared__ double red_d[4][AM_ROWS];
    __shared__ int red_c[4][AM_ROWS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int64_t row0 = (int64_t)blockIdx.x * AM_ROWS;
    const int64_t xr = min(row0 + col, rows - 1);  // rows past the end read the last row
    const float* xp = x + xr * HD + 4 * g;
    double bd[4];
    int bc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) { bd[e] = 0.0; bc[e] = -1; }

    for (int cg = 0; cg < C; cg += 256) {
        const CT* cp[4];
        int cid[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            cid[t] = cg + 64 * wave + 16 * t + col;
            cp[t] = centers + (int64_t)min(cid[t], C - 1) * HD + 4 * g;
        }
        f64x4 acc[4];
        double cc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) { acc[t] = f64x4{0.0, 0.0, 0.0, 0.0}; cc[t] = 0.0; }
        // a ring of AM_AHEAD k blocks of operands in flight (one k block =
        // 16 k: four MFMA steps per tile); block kb lives in slot kb % AM_AHEAD
        const int NB = HD / 16;
        u32x4 xa[AM_AHEAD];
        typename CP::V cb[AM_AHEAD][4];
        auto issue = [&](int kb, int slot) {
            xa[slot] = *reinterpret_cast<const u32x4*>(xp + 16 * kb);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                cb[slot][t] = *reinterpret_cast<const typename CP::V*>(cp[t] + 16 * kb);
        };
#pragma unroll
        for (int i = 0; i < AM_AHEAD; ++i)
            if (i < NB) issue(i, i);
        for (int kb0 = 0; kb0 < NB; kb0 += AM_AHEAD) {
#pragma unroll
            for (int i = 0; i < AM_AHEAD; ++i) {
                const int kb = kb0 + i;
                if (kb >= NB) break;
                const u32x4 xv = xa[i];
                typename CP::V cv[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) cv[t] = cb[i][t];
                if (kb + AM_AHEAD < NB) issue(kb + AM_AHEAD, i);
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const double a = (double)__uint_as_float(xv[st]);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const double b = CP::get(cv[t], st);
                        acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[t], 0, 0, 0);
                        cc[t] = fma(b, b, cc[t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            // ||c||^2 over the four k subsets of this column
            cc[t] += __shfl_xor(cc[t], 16);
            cc[t] += __shfl_xor(cc[t], 32);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double d = cc[t] - 2.0 * acc[t][e];
                const int c = cid[t] < C ? cid[t] : -1;
                if (better(d, c, bd[e], bc[e])) { bd[e] = d; bc[e] = c; }
            }
        }
    }
    // lanes of one row group (same g) hold rows 4e + g: reduce over columns
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const double od = __shfl_xor(bd[e], off);
            const int oc = __shfl_xor(bc[e], off);
            if (better(od, oc, bd[e], bc[e])) { bd[e] = od; bc[e] = oc; }
        }
    if (col == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            red_d[wave][4 * e + g] = bd[e];
            red_c[wave][4 * e + g] = bc[e];
        }
    }
    __syncthreads();
    if (threadIdx.x < AM_ROWS) {
        const int r = threadIdx.x;
        double d = red_d[0][r];
        int c = red_c[0][r];
        for (int w = 1; w < 4; ++w)
            if (better(red_d[w][r], red_c[w][r], d, c)) { d = red_d[w][r]; c = red_c[w][r]; }
        const int64_t gr = row0 + r;
        if (gr < rows) store_id<ID_BYTES>(ids, gr, c);
    }
}

// bf16 MFMA nearest-center search with an exact decision (C <= 256).
// x = hi + lo + r with hi = bf16(x), lo = bf16(x - hi), |r| <= 2^-16 |x|;
// the centers are exact bf16, so the two MFMA passes hi.c and lo.c have
// exact products and only fp32 sums.  The MFMA accumulator restarts every
// AB_SEG k values and the segment sums are added in a second fp32
// accumulator, so even with one fp32 rounding per addition the dot product
// is within (g_2SEG + g_nseg)(1 + 2^-7) + 2^-16 < 5e-5 of sum |x||c| <=
// ||x|| ||c|| (g_n = n 2^-24 / (1 - n 2^-24), nseg = HD / SEG <= 64);
// ||c||^2 is summed the same way (fp32 per segment, fp64 across: < 1e-5
// ||c||^2).  With the final fp32 subtraction every approximate distance
// dt_c = ||c||^2 - 2 x.c is within 1.1e-4 (||x|| ||c|| + ||c||^2) of the
// exact one (2e-4 if the matrix core truncated instead of rounding); the
// search uses
//   E_c = AB_KAPPA (||x|| ||c|| + ||c||^2),   AB_KAPPA = 2.5e-4,
// With U = min_c (dt_c + E_c) the exact argmin is among the candidates
// {c : dt_c - E_c <= U}; a row with one candidate is decided, a row with
// several re-evaluates just those in fp64 (exact products, first index on
// ties), the arithmetic of assign_kernel.
// A 512-thread block owns 32 rows; wave w takes centers 32w + [0, 32) as one
// 32 x 32 tile.  x is split into hi/lo bf16 tiles in LDS per 128-wide k
// chunk (shared by the eight waves); center fragments come from L2 one chunk
// ahead.  Needs HD % AB_SEG == 0, HD <= AB_MAXK, C <= 256, x and centers
// 16-byte aligned.
constexpr int AB_ROWS = 32, AB_KC = 128, AB_SEG = 256, AB_MAXC = 256, AB_WAVES = 8, AB_MAXK = 16384;
constexpr float AB_KAPPA = 2.5e-4f;

// ------------------------------------------------ batched encode problems
// One launch per encode stage serves up to ENC_MAXB independent problems of
// one shape (K and V of a layer, batch items): problem blockIdx.y (search,
// quantiser) or blockIdx.z (projection).  A problem's rows are fp32 (x) or
// bf16 (xb, read as the reference's value.float(): exact), row stride ldx.
constexpr int ENC_MAXB = 8;
struct EncProb {
    const float* x;
    const uint16_t* xb;
    int64_t ldx;
    const uint16_t* centers;
    void* ids;
    const float* mean;
    const uint16_t* w_enc;
    float* coeff;
    uint8_t* packed;
    uint16_t* scales;
    int64_t M;
};
struct EncBatch {
    EncProb p[ENC_MAXB];
    int n, K, r, num_centers, id_bytes;
    int64_t row_blocks;   // 32-row blocks of the largest problem (set per launch)
    // the quantiser run inside the projection: group size (0: separate
    // launch), scale dtype and NKV_QUANT_* mode
    int qgroup, scale_dtype, quant_mode;
    // center id of row m of problem p (clamped into the table)
    __device__ __forceinline__ int id_of(const EncProb& q, int64_t m) const {
        int v;
        if (id_bytes == 1) v = reinterpret_cast<const uint8_t*>(q.ids)[m];
        else if (id_bytes == 2) v = reinterpret_cast<const uint16_t*>(q.ids)[m];
        else v = reinterpret_cast<const int32_t*>(q.ids)[m];
        return min(max(v, 0), num_centers - 1);
    }
};

// Eight consecutive input values of one row (16-byte loads), held raw until
// they are used.
template <bool XB>
struct X8 {
    u32x4 w[XB ? 1 : 2];
    __device__ __forceinline__ void load(const EncProb& q, int64_t m, int k) {
        if constexpr (XB) {
            w[0] = *reinterpret_cast<const u32x4*>(q.xb + m * q.ldx + k);
        } else {
            const float* r = q.x + m * q.ldx + k;
            w[0] = *reinterpret_cast<const u32x4*>(r);
            w[1] = *reinterpret_cast<const u32x4*>(r + 4);
        }
    }
    __device__ __forceinline__ float operator[](int e) const {
        if constexpr (XB)
            return __uint_as_float((e & 1) ? (w[0][e >> 1] & 0xffff0000u) : (w[0][e >> 1] << 16));
        else
            return __uint_as_float(w[e >> 2][e & 3]);
    }
};

// Work item of block blk when a launch's items are cut into eight equal runs,
// one per XCD (blocks are dispatched to the XCDs round-robin): block blk runs
// slot blk / 8 of XCD blk % 8.  Items that share operands (one problem's
// centers, one W_enc column slice) are numbered together, so they meet in
// one XCD's L2.  Blocks past the last item get an item >= items.
__device__ __forceinline__ int64_t xcd_item(int64_t blk, int64_t items) {
    const int64_t per = (items + 7) >> 3;
    return (blk & 7) * per + (blk >> 3);
}
static inline unsigned xcd_grid(int64_t items) { return (unsigned)(8 * ((items + 7) >> 3)); }

// The quantiser over every problem of a batch (problem blockIdx.y).
template <int QUANT_MODE>
__global__ void __launch_bounds__(256) quant_pack_batch_kernel(EncBatch B, int group,
                                                               int scale_dtype) {
    const EncProb& P = B.p[blockIdx.y];
    quant_pack_group<QUANT_MODE>(P.coeff, P.M, B.r, group, scale_dtype, P.packed, P.scales,
                                 (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// The search's small block state: ||x||^2 per row, the per-wave bounds U,
// and each row's candidate count, first candidate and candidate bit set.
struct AssignSmall {
    float xn[AB_ROWS];
    float red[AB_WAVES][AB_ROWS];
    int cnt[AB_ROWS], first[AB_ROWS];
    uint32_t cand[AB_ROWS][AB_MAXC / 32];
};

__device__ __forceinline__ void assign_small_init(AssignSmall& sm, int t) {
    if (t < AB_ROWS) { sm.xn[t] = 0.0f; sm.cnt[t] = 0; sm.first[t] = 0x7fffffff; }
    for (int e = t; e < AB_ROWS * AB_MAXC / 32; e += 64 * AB_WAVES) (&sm.cand[0][0])[e] = 0u;
}

// The decision after the products: tot (this lane's 16 dot products x.c,
// rows 8(i/4) + 4hf + i%4 of the block, center col), cnf = ||c||^2, and
// sm.xn complete.  Rows with one candidate are decided; the others compare
// their candidates exactly in fp64 (one wave per row, lanes split HD).
template <int ID_BYTES, bool XB>
__device__ __forceinline__ void assign_finish(const EncBatch& B, const EncProb& P, AssignSmall& sm,
                                              const f32x16& tot, float cnf, int col, int64_t row0) {
    const int64_t rows = P.M;
    const int C = B.num_centers, HD = B.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    float dt[16], ee[16];
    {
        const float cnorm = sqrtf(cnf) * 1.001f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i / 4) + 4 * hf + (i % 4);
            const float xnorm = sqrtf(sm.xn[r]) * 1.001f;
            dt[i] = col < C ? cnf - 2.0f * tot[i] : INFINITY;
            ee[i] = AB_KAPPA * (xnorm * cnorm + cnf * 1.001f);
        }
    }
    // U = min over the row's columns of dt + E: a half-wave holds a row's 32 columns
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float u = dt[i] + ee[i];
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) u = fminf(u, __shfl_xor(u, off));
        if (l32 == 0) sm.red[wave][8 * (i / 4) + 4 * hf + (i % 4)] = u;
    }
    __syncthreads();
    // candidates: dt - E <= U
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i / 4) + 4 * hf + (i % 4);
        float U = sm.red[0][r];
#pragma unroll
        for (int w = 1; w < AB_WAVES; ++w) U = fminf(U, sm.red[w][r]);
        if (col < C && dt[i] - ee[i] <= U) {
            atomicAdd(&sm.cnt[r], 1);
            atomicMin(&sm.first[r], col);
            atomicOr(&sm.cand[r][col >> 5], 1u << (col & 31));
        }
    }
    __syncthreads();
    for (int r = wave; r < AB_ROWS; r += AB_WAVES) {
        const int64_t gr = row0 + r;
        if (gr >= rows) continue;
        // (no candidate only for non-finite rows: index 0 then)
        int best = sm.cnt[r] == 0 ? 0 : sm.first[r];
        if (sm.cnt[r] > 1) {
            double bd = 0.0;
            best = -1;
            for (int w = 0; w < AB_MAXC / 32; ++w) {
                uint32_t bits = sm.cand[r][w];
                while (bits) {
                    const int c = 32 * w + __builtin_ctz(bits);
                    bits &= bits - 1;
                    const uint16_t* cr = P.centers + (int64_t)c * HD;
                    double cc = 0.0, xc = 0.0;
                    // 8 consecutive values per lane and step (HD % 256 == 0), four
                    // steps' loads issued together, summed in ascending k
                    for (int k = 8 * lane; k < HD; k += 4 * 512) {
                        u32x4 cw[4];
                        X8<XB> x8[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if (k + 512 * u < HD) {
                                cw[u] = *reinterpret_cast<const u32x4*>(cr + k + 512 * u);
                                x8[u].load(P, gr, k + 512 * u);
                            }
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if (k + 512 * u >= HD) break;
                            const uint32_t w4[4] = {cw[u].x, cw[u].y, cw[u].z, cw[u].w};
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                const uint32_t hb = (e & 1) ? (w4[e >> 1] & 0xffff0000u) : (w4[e >> 1] << 16);
                                const double cv = (double)__uint_as_float(hb);
                                cc = fma(cv, cv, cc);
                                xc = fma((double)x8[u][e], cv, xc);
                            }
                        }
                    }
#pragma unroll
                    for (int off = 1; off < 64; off <<= 1) {
                        cc += __shfl_xor(cc, off);
                        xc += __shfl_xor(xc, off);
                    }
                    const double d = cc - 2.0 * xc;
                    if (best < 0 || d < bd) { bd = d; best = c; }  // ascending c: first index on ties
                }
            }
        }
        if (lane == 0) store_id<ID_BYTES>(P.ids, gr, best);
    }
}

template <int ID_BYTES, bool XB>
__global__ void __launch_bounds__(64 * AB_WAVES) assign_bf16_kernel(EncBatch B) {
    const EncProb& P = B.p[blockIdx.y];
    const int64_t rows = P.M;
    const int C = B.num_centers, HD = B.K;
    const uint16_t* __restrict__ centers = P.centers;
    if ((int64_t)blockIdx.x * AB_ROWS >= rows) return;
    __shared__ __align__(16) uint16_t xs[2][AB_ROWS][AB_KC + 8];
    __shared__ AssignSmall sm;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    const int64_t row0 = (int64_t)blockIdx.x * AB_ROWS;
    assign_small_init(sm, t);
    // fill: thread t splits row t/16, k columns 8*(t%16) .. +8 of each chunk
    const int frow = t >> 4, fk = 8 * (t & 15);
    const int64_t fr = min(row0 + frow, rows - 1);
    const bool frow_ok = row0 + frow < rows;
    // this lane's center column
    const int col = 32 * wave + l32;
    const uint16_t* crow = centers + (int64_t)min(col, C - 1) * HD + 8 * hf;
    f32x16 acc = {}, tot = {};
    float cseg = 0.0f;
    double cn = 0.0;
    float xsq = 0.0f;
    u32x4 bcur[8], bnxt[8];
    X8<XB> xcur, xnxt;
    auto fetch = [&](int kc, u32x4 (&b)[8], X8<XB>& xv) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) b[ks] = *reinterpret_cast<const u32x4*>(crow + kc + 16 * ks);
        xv.load(P, fr, kc + fk);
    };
    // one chunk: split x into hi / lo bf16 through LDS, then the MFMAs of
    // both passes and the column norms
    auto body = [&](int kc, const u32x4 (&bq)[8], const X8<XB>& xq) {
        {
            // split this thread's 8 values into hi / lo bf16
            const float v[8] = {xq[0], xq[1], xq[2], xq[3], xq[4], xq[5], xq[6], xq[7]};
            u32x4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t hp = pack_bf16x2(v[2 * e], v[2 * e + 1]);
                hi[e] = hp;
                lo[e] = pack_bf16x2(v[2 * e] - __uint_as_float(hp << 16),
                                    v[2 * e + 1] - __uint_as_float(hp & 0xffff0000u));
                xsq = fmaf(v[2 * e], v[2 * e], fmaf(v[2 * e + 1], v[2 * e + 1], xsq));
            }
            *reinterpret_cast<u32x4*>(&xs[0][frow][fk]) = hi;
            *reinterpret_cast<u32x4*>(&xs[1][frow][fk]) = lo;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&xs[0][l32][16 * ks + 8 * hf]);
            const bf16x8 al = *reinterpret_cast<const bf16x8*>(&xs[1][l32][16 * ks + 8 * hf]);
            const bf16x8 bb = as_bf16x8(bq[ks]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bb, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bb, acc, 0, 0, 0);
            // (the words go through named scalars: indexing the vector inside
            // the bit_cast was lowered to word 0 four times)
            const uint32_t w4[4] = {bq[ks].x, bq[ks].y, bq[ks].z, bq[ks].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bf16x2 wv = __builtin_bit_cast(bf16x2, w4[e]);
                cseg = __builtin_amdgcn_fdot2_f32_bf16(wv, wv, cseg, false);
            }
        }
        if ((kc + AB_KC) % AB_SEG == 0) {
            // end of a segment: fold it into the second accumulators
#pragma unroll
            for (int i = 0; i < 16; ++i) tot[i] += acc[i];
            acc = f32x16{};
            cn += (double)cseg;
            cseg = 0.0f;
        }
        __syncthreads();
    };
    // the next chunk's operands (the last chunk reloads itself), issued
    // before this chunk's work and kept there (the fence stops the scheduler
    // from sinking the loads next to their use)
    fetch(0, bcur, xcur);
    __syncthreads();
    for (int kc = 0; kc < HD; kc += AB_KC) {
        fetch(kc + AB_KC < HD ? kc + AB_KC : kc, bnxt, xnxt);
        __builtin_amdgcn_sched_barrier(0);
        body(kc, bcur, xcur);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) bcur[ks] = bnxt[ks];
        xcur = xnxt;
    }
    // ||x||^2 per row (16 threads per row), ||c||^2 per column (two k halves)
    atomicAdd(&sm.xn[frow], frow_ok ? xsq : 0.0f);
    cn += __shfl_xor(cn, 32);
    const float cnf = (float)cn;
    __syncthreads();
    assign_finish<ID_BYTES, XB>(B, P, sm, tot, cnf, col, row0);
}

// The same search for bf16 rows.  A bf16 x is its own hi part (lo = 0), so
// one MFMA pass gives the products the two-pass form gives, bit for bit.
// Both operands go global -> LDS by 1 KB DMA pieces in 128-wide k stages
// (72 KB: the 256 center rows and the block's 32 input rows, each as
// [row][16 chunks of 16 bytes] with chunk c of row q at slot c ^ (q % 8)),
// double-buffered: after the barrier of stage i the next stage is issued and
// stage i's 8 MFMAs per wave run under it; wave 0 also sums ||x||^2 of its
// fragments.  A block's stream is bound by a fixed cost per barrier plus one
// per 1 KB piece, so few large stages stream faster than many small ones (on
// the box 32 KB stages reached about 100 GB/s per CU, 8 KB stages 38 GB/s,
// whatever the number in flight).  The old form read every center fragment
// straight from L2 (32 rows per load instruction) and waited on it at every
// chunk.
constexpr int AD_KS = 128, AD_NST = 2;
constexpr int AD_CPR = AD_KS / 8;                 // 16-byte chunks per row
constexpr int AD_RPP = 1024 / (AD_KS * 2);        // rows per 1 KB piece
constexpr int AD_CPIECES = AB_MAXC / AD_RPP, AD_PIECES = AD_CPIECES + AB_ROWS / AD_RPP;
constexpr int AD_STAGE = AD_PIECES * 1024;
constexpr int AD_QLO = AD_PIECES / AB_WAVES, AD_NHI = AD_PIECES % AB_WAVES;
constexpr int AD_QMAX = AD_QLO + (AD_NHI ? 1 : 0);
constexpr int AD_SMEM = AD_NST * AD_STAGE;
static_assert(AD_SMEM + (int)sizeof(AssignSmall) <= 160 * 1024, "LDS budget");
static_assert(AB_SEG % AD_KS == 0, "segments are whole stages");
static_assert(AD_NST == 2, "the loop issues one stage ahead");

template <int ID_BYTES>
__global__ void __launch_bounds__(64 * AB_WAVES) assign_dma_kernel(EncBatch B) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ AssignSmall sm;
    // items: (problem, row block), row block fastest
    const int64_t item = xcd_item(blockIdx.x, B.n * B.row_blocks);
    if (item >= B.n * B.row_blocks) return;
    const EncProb& P = B.p[item / B.row_blocks];
    const int64_t rows = P.M;
    const int C = B.num_centers, HD = B.K, S = HD / AD_KS;
    const int64_t row0 = (item % B.row_blocks) * AB_ROWS;
    if (row0 >= rows) return;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hf = lane >> 5, l32 = lane & 31;
    assign_small_init(sm, t);
    // this wave's pieces e = wave + AB_WAVES i: center rows AD_RPP e .. (the
    // last row past C), then input rows (the last row past the end); lane L
    // brings slot L % AD_CPR of its row, logical chunk (L % AD_CPR) ^ (row % 8)
    const uint16_t* src[AD_QMAX];
#pragma unroll
    for (int i = 0; i < AD_QMAX; ++i) {
        const int e = wave + AB_WAVES * i;
        const int q = AD_RPP * e + lane / AD_CPR;          // row of the stage image
        const int ch = 8 * ((lane % AD_CPR) ^ (q & 7));
        if (e < AD_CPIECES) {
            src[i] = P.centers + (int64_t)min(q, C - 1) * HD + ch;
        } else {
            const int64_t m = min(row0 + (q - AB_MAXC), rows - 1);
            src[i] = P.xb + m * P.ldx + ch;
        }
    }
    auto issue = [&](int stg) {
        unsigned char* dst = smem_raw + (stg % AD_NST) * AD_STAGE;
#pragma unroll
        for (int i = 0; i < AD_QMAX; ++i)
            if (i < AD_QLO || wave < AD_NHI)
                dma16(src[i] + stg * AD_KS, dst + 1024 * (wave + AB_WAVES * i));
    };
    const int col = 32 * wave + l32;
    f32x16 acc = {}, tot = {};
    float cseg = 0.0f, xsq = 0.0f;
    double cn = 0.0;
    const int xrow_b = (AB_MAXC + l32) * (AD_KS * 2), crow_b = col * (AD_KS * 2);
    issue(0);
    for (int it = 0; it < S; ++it) {
        // stage it landed (nothing later is in flight yet), then the buffer
        // of stage it - 1 is free for stage it + 1
        wait_vmcnt<0>();
        lds_barrier();
        if (it + 1 < S) issue(it + 1);
        const unsigned char* sb = smem_raw + (it % AD_NST) * AD_STAGE;
        bf16x8 af[AD_KS / 16], cf[AD_KS / 16];
#pragma unroll
        for (int k16 = 0; k16 < AD_KS / 16; ++k16) {
            const int slot = 16 * ((2 * k16 + hf) ^ (l32 & 7));
            af[k16] = lds_b128(reinterpret_cast<const uint16_t*>(sb + xrow_b + slot));
            cf[k16] = lds_b128(reinterpret_cast<const uint16_t*>(sb + crow_b + slot));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k16 = 0; k16 < AD_KS / 16; ++k16) {
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[k16], cf[k16], acc, 0, 0, 0);
            const u32x4 cw = __builtin_bit_cast(u32x4, cf[k16]);
            const uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bf16x2 wv = __builtin_bit_cast(bf16x2, w4[e]);
                cseg = __builtin_amdgcn_fdot2_f32_bf16(wv, wv, cseg, false);
            }
            if (wave == 0) {
                const u32x4 xw = __builtin_bit_cast(u32x4, af[k16]);
                const uint32_t x4[4] = {xw.x, xw.y, xw.z, xw.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bf16x2 xv = __builtin_bit_cast(bf16x2, x4[e]);
                    xsq = __builtin_amdgcn_fdot2_f32_bf16(xv, xv, xsq, false);
                }
            }
        }
        if (((it + 1) * AD_KS) % AB_SEG == 0 || it + 1 == S) {
            // end of a segment: fold it into the second accumulators
#pragma unroll
            for (int i = 0; i < 16; ++i) tot[i] += acc[i];
            acc = f32x16{};
            cn += (double)cseg;
            cseg = 0.0f;
        }
    }
    // ||x||^2 per row (wave 0: two k halves), ||c||^2 per column (two k halves)
    if (wave == 0) {
        const float xs2 = xsq + __shfl_xor(xsq, 32);
        if (hf == 0 && row0 + l32 < rows) sm.xn[l32] = xs2;
    }
    cn += __shfl_xor(cn, 32);
    __syncthreads();
    assign_finish<ID_BYTES, true>(B, P, sm, tot, (float)cn, col, row0);
}

// ============================================================ MFMA GEMM core
// C[M, N] = A[M, K] * B[N, K]^T on v_mfma_f32_32x32x16_bf16.  A 256-thread
// block computes a 64 x 64 tile: wave w owns the 32 x 32 sub-tile
// (w / 2, w % 2).  K advances in steps of 32 through LDS.
//
// 32x32x16 operand layout (wave64): lane l supplies row (l % 32) of A and
// column (l % 32) of B, with k = 8 * (l / 32) + [0, 8) inside the 16-wide
// step.  The 16 accumulator values of lane l belong to column (l % 32) and
// rows 8 * (i / 4) + 4 * (l / 32) + (i % 4).
constexpr int GT_M = 64, GT_N = 64, GT_K = 32, GT_PAD = 8;

struct GemmSmem {
    uint16_t a[GT_M][GT_K + GT_PAD];
    uint16_t b[GT_N][GT_K + GT_PAD];
};

__device__ __forceinline__ bf16x8 lds_bf16x8(const uint16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
}

// Encoder A-tile loader: A[m, k] = bf16(x[m, k] - center[id[m], k] - mean[k]).
struct EncodeA {
    const float* x;
    const uint16_t* centers;
    const void* ids;
    int id_bytes;
    int num_centers;
    const float* mean;
    int64_t M;
    int K;
    __device__ __forceinline__ int id_of(int64_t m) const {
        int v;
        if (id_bytes == 1) v = reinterpret_cast<const uint8_t*>(ids)[m];
        else if (id_bytes == 2) v = reinterpret_cast<const uint16_t*>(ids)[m];
        else v = reinterpret_cast<const int32_t*>(ids)[m];
        return min(max(v, 0), num_centers - 1);
    }
    // thread t fills row t/4, k-columns (t%4)*8 .. +8 of the 64 x 32 tile
    __device__ __forceinline__ void load(GemmSmem& s, int64_t m0, int k0, int t) const {
        const int rr = t / 4, kc = (t % 4) * 8;
        const int64_t m = m0 + rr;
        u32x4 packedv = {0, 0, 0, 0};
        if (m < M) {
            const float* xp = x + m * K + k0 + kc;
            f32x4 x0 = *reinterpret_cast<const f32x4*>(xp);
            f32x4 x1 = *reinterpret_cast<const f32x4*>(xp + 4);
            float v[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            if (centers) {
                const uint16_t* cp = centers + (int64_t)id_of(m) * K + k0 + kc;
                u32x4 cw = *reinterpret_cast<const u32x4*>(cp);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] = v[2 * e] - __uint_as_float(cw[e] << 16);
                    v[2 * e + 1] = v[2 * e + 1] - __uint_as_float(cw[e] & 0xffff0000u);
                }
            }
            if (mean) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = v[e] - mean[k0 + kc + e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) packedv[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
        }
        *reinterpret_cast<u32x4*>(&s.a[rr][kc]) = packedv;
    }
};

// Decoder A-tile loader: A[m, k] = bf16(code * scale) of row src(m).
struct DecodeA {
    const uint8_t* packed;
    const uint16_t* scales;
    const int32_t* row_index;
    int scale_dtype;
    int group;
    int64_t M;   // output rows
    int K;       // r
    __device__ __forceinline__ void load(GemmSmem& s, int64_t m0, int k0, int t) const {
        const int rr = t / 4, kc = (t % 4) * 8;
        const int64_t m = m0 + rr;
        u32x4 o = {0, 0, 0, 0};
        if (m < M) {
            const int64_t src = row_index ? (int64_t)row_index[m] : m;
            const uint32_t word =
                *reinterpret_cast<const uint32_t*>(packed + src * (K / 2) + (k0 + kc) / 2);
            const float sc =
                scale_bits_to_f32(scales[src * (K / group) + (k0 + kc) / group], scale_dtype);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float lo = (float)((int)((word >> (8 * e)) & 15u) - 7) * sc;
                float hi = (float)((int)((word >> (8 * e + 4)) & 15u) - 7) * sc;
                o[e] = pack_bf16x2(lo, hi);
            }
        }
        *reinterpret_cast<u32x4*>(&s.a[rr][kc]) = o;
    }
};

// B tile [64 rows (n) x 32 k] of a bf16 row-major [N, K] matrix.
__device__ __forceinline__ void load_b_tile(GemmSmem& s, const uint16_t* __restrict__ B,
                                            int64_t N, int K, int64_t n0, int k0, int t) {
    const int rr = t / 4, kc = (t % 4) * 8;
    const int64_t n = n0 + rr;
    u32x4 v = {0, 0, 0, 0};
    if (n < N) v = *reinterpret_cast<const u32x4*>(B + n * K + k0 + kc);
    *reinterpret_cast<u32x4*>(&s.b[rr][kc]) = v;
}

template <class ALoader>
__device__ __forceinline__ f32x16 gemm_tile(GemmSmem& s, const ALoader& al,
                                            const uint16_t* __restrict__ B, int64_t N, int K,
                                            int64_t m0, int64_t n0) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int hf = lane >> 5, l32 = lane & 31;
    f32x16 acc = {};
    for (int k0 = 0; k0 < K; k0 += GT_K) {
        __syncthreads();
        al.load(s, m0, k0, t);
        load_b_tile(s, B, N, K, n0, k0, t);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < GT_K; kk += 16) {
            bf16x8 a = lds_bf16x8(&s.a[wm + l32][kk + 8 * hf]);
            bf16x8 b = lds_bf16x8(&s.b[wn + l32][kk + 8 * hf]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
    }
    return acc;
}

__global__ void __launch_bounds__(256) encode_gemm_kernel(EncodeA al,
                                                          const uint16_t* __restrict__ w_enc,
                                                          int r, float* __restrict__ coeff) {
    __shared__ GemmSmem s;
    const int64_t m0 = (int64_t)blockIdx.x * GT_M, n0 = (int64_t)blockIdx.y * GT_N;
    f32x16 acc = gemm_tile(s, al, w_enc, r, al.K, m0, n0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    const int64_t n = n0 + (wave & 1) * 32 + l32;
    if (n >= r) return;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t m = m0 + (wave >> 1) * 32 + 8 * (i / 4) + 4 * hf + (i % 4);
        if (m < al.M) coeff[m * r + n] = acc[i];
    }
}

// Encoder projection coeff[M, r] = bf16(x - center[id] - mean) W_enc^T, fp32
// accumulation (MG nanokv_codec.py:344-347: the residual minus the mean, in
// bf16, through the bf16 operator).  A block of six waves owns 32 rows x 192
// coefficient columns (wave w: columns 32w .. 32w + 32) and walks K in
// 128-wide stages.  Every operand goes global -> LDS by 1 KB DMA pieces,
// double-buffered (no register staging, so no wait covers more than the
// stage it needs):
//   [W_enc 192 rows x 256 B][inputs 32 rows][center values 32 rows][mean]
// (the mean piece holds the stage's 128 means twice).  Stage i: wait, barrier,
// issue stage i + 1, waves 0-3 turn stage i into the bf16 residual image (two
// 16-byte units of one row per thread), barrier, 8 MFMAs per wave.  A block's
// stream is bound by a fixed cost per barrier plus one per piece, so few
// large stages stream faster than many small ones (64-wide stages four deep
// took 34.5-39.6 us for a 1,560-row K+V chunk).  W and the residual image are
// [row][16 chunks of 16 bytes] with chunk c of row q at slot c ^ (q % 8), so
// the operand reads (32 rows at one chunk) are free of bank conflicts.  Needs
// K % 128 == 0 and 16-byte aligned rows.
constexpr int EP_ROWS = 32, EP_WAVES = 6, EP_COLS = 32 * EP_WAVES, EP_KS = 128;
constexpr int EP_CPR = EP_KS / 8;                  // 16-byte chunks per bf16 row
constexpr int EP_RPP = 1024 / (EP_KS * 2);         // bf16 rows per 1 KB piece
constexpr int EP_WPIECES = EP_COLS / EP_RPP;

template <bool XB>
struct EncProjFmt {
    static constexpr int XROW = EP_KS * (XB ? 2 : 4);               // input bytes per row
    static constexpr int XPIECES = EP_ROWS * XROW / 1024;
    static constexpr int X0 = EP_WPIECES, C0 = X0 + XPIECES, M0 = C0 + EP_ROWS / EP_RPP;
    static constexpr int PIECES = M0 + 1;
    static constexpr int STAGE = PIECES * 1024;                      // bytes
    static constexpr int AIMG = EP_ROWS * EP_KS * 2;                 // residual image bytes
    static constexpr int SMEM = 2 * STAGE + AIMG;
    // pieces per wave and stage: the first PIECES % EP_WAVES waves take one more
    static constexpr int QLO = PIECES / EP_WAVES, NHI = PIECES % EP_WAVES;
    static constexpr int QMAX = QLO + (NHI ? 1 : 0);
};

template <bool XB>
__global__ void __launch_bounds__(64 * EP_WAVES) encode_proj_kernel(EncBatch B) {
    using F = EncProjFmt<XB>;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    // items: (problem, column slice, row block), row block fastest
    const int ncb = (B.r + EP_COLS - 1) / EP_COLS;
    const int64_t item = xcd_item(blockIdx.x, B.n * ncb * B.row_blocks);
    if (item >= B.n * ncb * B.row_blocks) return;
    const int64_t rest = item / B.row_blocks;
    const EncProb& P = B.p[rest / ncb];
    const int r = B.r, K = B.K, S = K / EP_KS;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hf = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (item % B.row_blocks) * EP_ROWS;
    if (m0 >= P.M) return;
    const int n0 = (int)(rest % ncb) * EP_COLS;
    // this wave's pieces e = wave + EP_WAVES i: per lane a source address
    // and the bytes it advances per stage.  Rows past the end read the last
    // row; absent centers or mean read W_enc (any readable bytes; unused).
    const unsigned char* src[F::QMAX];
    int64_t adv[F::QMAX];
    auto xrow = [&](int q) { return min(m0 + q, P.M - 1); };
#pragma unroll
    for (int i = 0; i < F::QMAX; ++i) {
        const int e = wave + EP_WAVES * i;
        const unsigned char* sp = reinterpret_cast<const unsigned char*>(P.w_enc);
        int64_t st = 0;
        if (e < F::X0) {
            // W row n0 + q, slot lane % EP_CPR holds chunk slot ^ (q % 8)
            const int q = EP_RPP * e + lane / EP_CPR;
            const int row = min(n0 + q, r - 1);
            sp = reinterpret_cast<const unsigned char*>(P.w_enc + (int64_t)row * K +
                                                        8 * ((lane % EP_CPR) ^ (q & 7)));
            st = 2 * EP_KS;
        } else if (e < F::C0) {
            constexpr int CPRX = F::XROW / 16, RPPX = 1024 / F::XROW;
            const int64_t m = xrow(RPPX * (e - F::X0) + lane / CPRX);
            const int off = 16 * (lane % CPRX);
            sp = XB ? reinterpret_cast<const unsigned char*>(P.xb + m * P.ldx) + off
                    : reinterpret_cast<const unsigned char*>(P.x + m * P.ldx) + off;
            st = F::XROW;
        } else if (e < F::M0) {
            if (P.centers) {
                const int64_t m = xrow(EP_RPP * (e - F::C0) + lane / EP_CPR);
                sp = reinterpret_cast<const unsigned char*>(P.centers + (int64_t)B.id_of(P, m) * K +
                                                            8 * (lane % EP_CPR));
                st = 2 * EP_KS;
            }
        } else if (e == F::M0) {
            if (P.mean) {
                sp = reinterpret_cast<const unsigned char*>(P.mean + 4 * (lane % (EP_KS / 4)));
                st = 4 * EP_KS;
            }
        }
        src[i] = sp;
        adv[i] = st;
    }
    auto issue = [&](int stg) {
        unsigned char* dst = smem_raw + (stg & 1) * F::STAGE;
#pragma unroll
        for (int i = 0; i < F::QMAX; ++i) {
            const int e = wave + EP_WAVES * i;
            if (i < F::QLO || wave < F::NHI) dma16(src[i] + stg * adv[i], dst + 1024 * e);
        }
    };
    unsigned char* aimg = smem_raw + 2 * F::STAGE;
    const bool prod = wave < 4;
    // stage stg (landed) -> the residual image; absent centers or mean
    // subtract zeros (x - 0 = x exactly), so every read is unconditional
    const bool has_c = P.centers != nullptr, has_m = P.mean != nullptr;
    auto prep = [&](int stg) {
        const unsigned char* sb = smem_raw + (stg & 1) * F::STAGE;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int unit = t + 256 * u;                       // of 32 rows x 16 chunks
            const int arow = unit / EP_CPR, ach = unit % EP_CPR;
            const u32x4 c = *reinterpret_cast<const u32x4*>(sb + 1024 * F::C0 + arow * (EP_KS * 2) + 16 * ach);
            const f32x4* mp = reinterpret_cast<const f32x4*>(sb + 1024 * F::M0 + 32 * ach);
            const f32x4 u0 = mp[0], u1 = mp[1];
            float xv[8];
            if constexpr (XB) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(sb + 1024 * F::X0 + arow * F::XROW + 16 * ach);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xv[2 * e] = __uint_as_float(w[e] << 16);
                    xv[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
                }
            } else {
                const f32x4* xp = reinterpret_cast<const f32x4*>(sb + 1024 * F::X0 + arow * F::XROW + 32 * ach);
                const f32x4 a0 = xp[0], a1 = xp[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) { xv[e] = a0[e]; xv[4 + e] = a1[e]; }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t cw = (e & 1) ? (c[e >> 1] & 0xffff0000u) : (c[e >> 1] << 16);
                const float cv = has_c ? __uint_as_float(cw) : 0.0f;
                const float mv = has_m ? (e < 4 ? u0[e] : u1[e - 4]) : 0.0f;
                xv[e] = (xv[e] - cv) - mv;
            }
            const bool ok = m0 + arow < P.M;
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = ok ? pack_bf16x2(xv[2 * e], xv[2 * e + 1]) : 0u;
            *reinterpret_cast<u32x4*>(aimg + arow * (EP_KS * 2) + 16 * (ach ^ (arow & 7))) = o;
        }
    };
    const bool cols = n0 + 32 * wave < r;
    f32x16 acc = {};
    const int arow_b = l32 * (EP_KS * 2), wrow_b = (32 * wave + l32) * (EP_KS * 2);
    auto compute = [&](int stg) {
        const unsigned char* wr = smem_raw + (stg & 1) * F::STAGE + wrow_b;
        bf16x8 af[EP_KS / 16], wf[EP_KS / 16];
#pragma unroll
        for (int k16 = 0; k16 < EP_KS / 16; ++k16) {
            const int slot = 16 * ((2 * k16 + hf) ^ (l32 & 7));
            af[k16] = lds_b128(reinterpret_cast<const uint16_t*>(aimg + arow_b + slot));
            wf[k16] = lds_b128(reinterpret_cast<const uint16_t*>(wr + slot));
        }
        // all reads in flight before the first product
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k16 = 0; k16 < EP_KS / 16; ++k16)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[k16], wf[k16], acc, 0, 0, 0);
    };
    issue(0);
    for (int it = 0; it < S; ++it) {
        // stage it landed (nothing later is in flight yet); after the barrier
        // every wave is past stage it - 1, whose buffer takes stage it + 1
        wait_vmcnt<0>();
        lds_barrier();
        if (it + 1 < S) issue(it + 1);
        if (prod) prep(it);
        lds_barrier();
        if (cols) compute(it);
    }
    const int n = n0 + 32 * wave + l32;
    if (cols && n < r) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t mm = m0 + 8 * (i / 4) + 4 * hf + (i % 4);
            if (mm < P.M) P.coeff[mm * r + n] = acc[i];
        }
    }
    if (B.qgroup == 0) return;
    // the quantiser on the block's whole groups (the columns of a block hold
    // whole groups): the coefficients just stored, read back after the barrier
    __syncthreads();
    const int G = B.qgroup, ngroups = r / G, gpb = (min(r - n0, EP_COLS)) / G;
    for (int it = t; it < EP_ROWS * gpb; it += 64 * EP_WAVES) {
        const int64_t gid = (m0 + it / gpb) * ngroups + n0 / G + it % gpb;
        if (B.quant_mode == NKV_QUANT_BF16)
            quant_pack_group<NKV_QUANT_BF16>(P.coeff, P.M, r, G, B.scale_dtype, P.packed, P.scales, gid);
        else
            quant_pack_group<NKV_QUANT_FP32>(P.coeff, P.M, r, G, B.scale_dtype, P.packed, P.scales, gid);
    }
}

// Dynamic LDS of the projection kernels (above 64 KB), set once per process.
static int encode_proj_smem() {
    static const int rc = [] {
        const hipError_t e0 = hipFuncSetAttribute((const void*)encode_proj_kernel<true>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  EncProjFmt<true>::SMEM);
        const hipError_t e1 = hipFuncSetAttribute((const void*)encode_proj_kernel<false>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  EncProjFmt<false>::SMEM);
        return e0 == hipSuccess && e1 == hipSuccess ? (int)NKV_OK : (int)NKV_ERR_HIP;
    }();
    return rc;
}
static_assert(EncProjFmt<false>::SMEM <= 160 * 1024, "LDS budget");

struct DecodeEpi {
    const uint16_t* centers;   // [C, HD] for this batch item, or NULL
    const void* ids;           // [N] of this batch item
    int id_bytes;
    int num_centers;
    const int32_t* row_index;
    const float* mean;
    // ids outside the table are clamped (a corrupt payload must not read out of bounds)
    __device__ __forceinline__ int id_of(int64_t src) const {
        int v;
        if (id_bytes == 1) v = reinterpret_cast<const uint8_t*>(ids)[src];
        else if (id_bytes == 2) v = reinterpret_cast<const uint16_t*>(ids)[src];
        else v = reinterpret_cast<const int32_t*>(ids)[src];
        return min(max(v, 0), num_centers - 1);
    }
};

// out[m, n] = bf16(bf16(acc + bf16(mean[n])) + center[id[src(m)], n])   (MG:438-454)
__global__ void __launch_bounds__(256) decode_gemm_kernel(DecodeA al, DecodeEpi ep,
                                                          const uint16_t* __restrict__ w_dec,
                                                          int HD, uint16_t* __restrict__ out) {
    __shared__ GemmSmem s;
    const int64_t m0 = (int64_t)blockIdx.x * GT_M, n0 = (int64_t)blockIdx.y * GT_N;
    f32x16 acc = gemm_tile(s, al, w_dec, HD, al.K, m0, n0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    const int64_t n = n0 + (wave & 1) * 32 + l32;
    if (n >= HD) return;
    const float bias = ep.mean ? bf16_round(ep.mean[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t m = m0 + (wave >> 1) * 32 + 8 * (i / 4) + 4 * hf + (i % 4);
        if (m >= al.M) continue;
        float v = bf16_round(acc[i] + bias);
        if (ep.centers) {
            const int64_t src = ep.row_index ? (int64_t)ep.row_index[m] : m;
            v = bf16_round(v + bf16_bits_to_f32(ep.centers[(int64_t)ep.id_of(src) * HD + n]));
        }
        out[m * HD + n] = f32_to_bf16_bits(v);
    }
}

}  // namespace nkv

using namespace nkv;

// ============================================================ C ABI
static int check_codec_layout(int r, int group, int scale_dtype) {
    NKV_REQUIRE(r > 0 && r % 32 == 0, NKV_ERR_INVALID, "r must be a positive multiple of 32");
    NKV_REQUIRE(group > 0 && r % group == 0 && group % 8 == 0, NKV_ERR_INVALID,
                "group must divide r and be a multiple of 8");
    NKV_REQUIRE(scale_dtype == NKV_DTYPE_BF16 || scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "scale_dtype must be NKV_DTYPE_BF16 or NKV_DTYPE_FP16");
    return NKV_OK;
}

namespace nkv {

// ------------------------------------------------------- INT8 operator weights
// _pack_operator (MG:108-131): per (row, group) s = max(amax|w|, 1e-12) / 127
// in fp32, q = clamp(rint(w / s), -127, 127), stored scale = bf16(s) (the codes
// use the unrounded s).  One wave per (row, group): a wave-wide amax, then
// every lane codes elements lane, lane + 64, ...
__global__ void __launch_bounds__(256) int8_pack_kernel(const float* __restrict__ w, int64_t rows,
                                                        int cols, int group,
                                                        int8_t* __restrict__ q,
                                                        uint16_t* __restrict__ scale) {
    const int lane = threadIdx.x & 63;
    const int ngroups = cols / group;
    const int64_t gid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gid >= rows * ngroups) return;  // uniform per wave
    const int64_t row = gid / ngroups;
    const int64_t base = row * cols + (gid - row * ngroups) * (int64_t)group;
    float amax = 0.0f;
    for (int j = lane; j < group; j += 64) {
        const float a = fabsf(w[base + j]);
        amax = (a > amax || a != a) ? a : amax;  // NaN propagates like torch.amax
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float b = __shfl_xor(amax, o);
        amax = (b > amax || b != b) ? b : amax;
    }
    const float s = __fdiv_rn((amax > 1e-12f || amax != amax) ? amax : 1e-12f, 127.0f);
    if (lane == 0) scale[gid] = f32_to_bf16_bits(s);
    for (int j = lane; j < group; j += 64) {
        const float r = rintf(__fdiv_rn(w[base + j], s));  // round half to even (torch.round)
        q[base + j] = (int8_t)(int)fminf(fmaxf(r, -127.0f), 127.0f);
    }
}

// unpack_int8_weight (nanokv_codec_kernels.py:64-82), _operator_linear
// (MG:145-152): out = bf16(q * scale); the product of an 8-bit integer and a
// bf16 scale is exact in fp32, so out is rounded once.  Eight weights per
// thread when the row length allows 8-byte loads.
__global__ void __launch_bounds__(256) int8_dequant_kernel(const int8_t* __restrict__ q,
                                                           const uint16_t* __restrict__ scale,
                                                           int64_t count, int group,
                                                           uint16_t* __restrict__ out) {
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i0 >= count) return;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t i = i0 + e;
        if (i < count)
            out[i] = f32_to_bf16_bits((float)q[i] * bf16_bits_to_f32(scale[i / group]));
    }
}

}  // namespace nkv

extern "C" int nkv_quant_pack(void* stream, const float* coeff, int64_t rows, int r, int group,
                              int scale_dtype, int quant_mode, uint8_t* packed,
                              uint16_t* scales) {
    clear_error();
    NKV_REQUIRE(rows >= 0, NKV_ERR_INVALID, "rows must be >= 0");
    NKV_REQUIRE(r > 0 && r % 8 == 0, NKV_ERR_INVALID, "r must be a positive multiple of 8");
    NKV_REQUIRE(group > 0 && r % group == 0 && group % 8 == 0, NKV_ERR_INVALID,
                "group must divide r and be a multiple of 8");
    NKV_REQUIRE(scale_dtype == NKV_DTYPE_BF16 || scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    NKV_REQUIRE(quant_mode == NKV_QUANT_FP32 || quant_mode == NKV_QUANT_BF16, NKV_ERR_INVALID,
                "bad quant_mode");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(coeff && packed && scales, NKV_ERR_INVALID, "null pointer");
    const int64_t threads = rows * (r / group);
    dim3 grid((unsigned)cdiv(threads, 256));
    hipStream_t s = (hipStream_t)stream;
    if (quant_mode == NKV_QUANT_BF16)
        quant_pack_kernel<NKV_QUANT_BF16><<<grid, 256, 0, s>>>(coeff, rows, r, group, scale_dtype,
                                                                packed, scales);
    else
        quant_pack_kernel<NKV_QUANT_FP32><<<grid, 256, 0, s>>>(coeff, rows, r, group, scale_dtype,
                                                                packed, scales);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

extern "C" int nkv_int8_pack(void* stream, const float* w, int64_t rows, int cols, int group,
                             int8_t* q, uint16_t* scale) {
    clear_error();
    NKV_REQUIRE(rows >= 0 && cols > 0, NKV_ERR_INVALID, "bad weight shape");
    NKV_REQUIRE(group > 0 && cols % group == 0, NKV_ERR_INVALID, "group must divide cols");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(w && q && scale, NKV_ERR_INVALID, "null pointer");
    const int64_t waves = rows * (cols / group);
    nkv::int8_pack_kernel<<<dim3((unsigned)cdiv(waves, 4)), 256, 0, (hipStream_t)stream>>>(
        w, rows, cols, group, q, scale);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

extern "C" int nkv_int8_dequant(void* stream, const int8_t* q, const uint16_t* scale, int64_t rows,
                                int cols, int group, uint16_t* out) {
    clear_error();
    NKV_REQUIRE(rows >= 0 && cols > 0, NKV_ERR_INVALID, "bad weight shape");
    NKV_REQUIRE(group > 0 && cols % group == 0, NKV_ERR_INVALID, "group must divide cols");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(q && scale && out, NKV_ERR_INVALID, "null pointer");
    const int64_t count = rows * cols;
    nkv::int8_dequant_kernel<<<dim3((unsigned)cdiv(cdiv(count, 8), 256)), 256, 0,
                               (hipStream_t)stream>>>(q, scale, count, group, out);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

extern "C" int nkv_unpack(void* stream, const uint8_t* packed, const uint16_t* scales,
                          int scale_dtype, const int32_t* row_index, int64_t rows, int r,
                          int group, uint16_t* latent) {
    clear_error();
    NKV_REQUIRE(rows >= 0, NKV_ERR_INVALID, "rows must be >= 0");
    NKV_REQUIRE(r > 0 && r % 8 == 0, NKV_ERR_INVALID, "r must be a positive multiple of 8");
    NKV_REQUIRE(group > 0 && r % group == 0 && group % 8 == 0, NKV_ERR_INVALID,
                "group must divide r and be a multiple of 8");
    NKV_REQUIRE(scale_dtype == NKV_DTYPE_BF16 || scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(packed && scales && latent, NKV_ERR_INVALID, "null pointer");
    const int64_t threads = rows * (r / 8);
    unpack_kernel<<<dim3((unsigned)cdiv(threads, 256)), 256, 0, (hipStream_t)stream>>>(
        packed, scales, scale_dtype, row_index, rows, r, group, latent);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

namespace nkv {

// ------------------------------------------------------------ C64 fit
// The per-chunk joint-head center fit of semantic_residual (MG:301-330):
// centers start as the rows init_rows (the caller's seeded permutation),
// then each round labels every row with its nearest center (the exact fp64
// search, first index on ties) and moves every center that has rows to their
// mean.  The mean is deterministic: the rows of each cluster are listed in
// row order (a stable counting sort), summed in fp64 in that order, rounded
// to fp32 and divided by the count in fp32.

__global__ void __launch_bounds__(256) c64_init_kernel(const float* __restrict__ x, int B, int64_t S,
                                                       int HD, int C,
                                                       const int32_t* __restrict__ init_rows,
                                                       float* __restrict__ centers) {
    const int64_t total = (int64_t)B * C * HD;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % HD);
        const int c = (int)((i / HD) % C);
        const int64_t b = i / ((int64_t)HD * C);
        const int64_t row = min(max((int64_t)init_rows[c], (int64_t)0), S - 1);
        centers[i] = x[(b * S + row) * HD + d];
    }
}

constexpr int FIT_THREADS = 256, FIT_MAXC = 256;

// One block per batch item: cluster sizes, their exclusive offsets, and the
// rows of each cluster in row order (order[offset[c] + k] = k-th row of c).
__global__ void __launch_bounds__(FIT_THREADS) c64_sort_kernel(const int32_t* __restrict__ labels,
                                                                int64_t S, int C,
                                                                int32_t* __restrict__ counts,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ order) {
    __shared__ int cnt[FIT_MAXC], cur[FIT_MAXC], lab[FIT_THREADS];
    const int t = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int32_t* lb = labels + b * S;
    for (int c = t; c < C; c += FIT_THREADS) cnt[c] = 0;
    __syncthreads();
    for (int64_t i = t; i < S; i += FIT_THREADS) atomicAdd(&cnt[min(max(lb[i], 0), C - 1)], 1);
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int c = 0; c < C; ++c) {
            cur[c] = run;
            run += cnt[c];
        }
    }
    __syncthreads();
    for (int c = t; c < C; c += FIT_THREADS) {
        counts[b * C + c] = cnt[c];
        offsets[b * C + c] = cur[c];
    }
    for (int64_t i0 = 0; i0 < S; i0 += FIT_THREADS) {
        const int64_t i = i0 + t;
        const int L = i < S ? min(max(lb[i], 0), C - 1) : -1;
        lab[t] = L;
        __syncthreads();
        if (L >= 0) {
            // rows of this cluster earlier in the chunk come first
            int rank = 0;
            for (int u = 0; u < t; ++u) rank += lab[u] == L;
            order[b * S + cur[L] + rank] = (int32_t)i;
        }
        __syncthreads();
        if (L >= 0) atomicAdd(&cur[L], 1);
        __syncthreads();
    }
}

// grid (cdiv(HD, 256), C, B): one thread per center element.
__global__ void __launch_bounds__(256) c64_update_kernel(const float* __restrict__ x, int64_t S,
                                                         int HD, int C,
                                                         const int32_t* __restrict__ counts,
                                                         const int32_t* __restrict__ offsets,
                                                         const int32_t* __restrict__ order,
                                                         float* __restrict__ centers) {
    const int d = blockIdx.x * 256 + threadIdx.x;
    const int c = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (d >= HD) return;
    const int n = counts[b * C + c];
    if (n == 0) return;  // an empty cluster keeps its center
    const int32_t* ord = order + b * S + offsets[b * C + c];
    const float* xb = x + b * S * HD + d;
    double sum = 0.0;
    for (int k = 0; k < n; ++k) sum += (double)xb[(int64_t)ord[k] * HD];
    centers[(b * C + c) * HD + d] = __fdiv_rn((float)sum, (float)n);
}

__global__ void zero_i32_kernel(int32_t* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace nkv

// Nearest fp32 center of every row (int32 labels): the fp64 MFMA search, or
// the fp64 VALU search for unaligned operands.
static int launch_assign_f32(hipStream_t s, const float* x, const float* centers, int64_t rows,
                             int C, int HD, int32_t* ids) {
    if (rows <= 0) return NKV_OK;
    if (HD % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(centers) % 16 == 0) {
        assign_mfma_kernel<4, float><<<dim3((unsigned)cdiv(rows, AM_ROWS)), 256, 0, s>>>(
            x, centers, rows, C, HD, ids);
    } else {
        assign_kernel<4, float><<<dim3((unsigned)cdiv(rows, AS_ROWS)), 256, 0, s>>>(
            x, centers, rows, C, HD, ids);
    }
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

// The exact bf16-MFMA nearest-center search over every problem of a batch
// (C <= AB_MAXC, HD % AB_SEG == 0, HD <= AB_MAXK, 16-byte aligned rows).
static int launch_assign_batch(hipStream_t s, EncBatch B, bool xb) {
    int64_t rows = 0;
    for (int i = 0; i < B.n; ++i) rows = std::max(rows, B.p[i].M);
    if (rows <= 0) return NKV_OK;
    B.row_blocks = cdiv(rows, AB_ROWS);
    const dim3 grid((unsigned)cdiv(rows, AB_ROWS), (unsigned)B.n);
    const unsigned threads = 64 * AB_WAVES;
    if (xb) {
        static const hipError_t attr = [] {
            hipError_t e = hipSuccess;
            for (const void* f : {(const void*)assign_dma_kernel<1>, (const void*)assign_dma_kernel<2>,
                                  (const void*)assign_dma_kernel<4>})
                if (e == hipSuccess)
                    e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, AD_SMEM);
            return e;
        }();
        NKV_REQUIRE(attr == hipSuccess, NKV_ERR_HIP, "hipFuncSetAttribute failed for the search kernels");
        const unsigned g1 = xcd_grid(B.n * B.row_blocks);
        if (B.id_bytes == 1) assign_dma_kernel<1><<<g1, threads, AD_SMEM, s>>>(B);
        else if (B.id_bytes == 2) assign_dma_kernel<2><<<g1, threads, AD_SMEM, s>>>(B);
        else assign_dma_kernel<4><<<g1, threads, AD_SMEM, s>>>(B);
    } else {
        if (B.id_bytes == 1) assign_bf16_kernel<1, false><<<grid, threads, 0, s>>>(B);
        else if (B.id_bytes == 2) assign_bf16_kernel<2, false><<<grid, threads, 0, s>>>(B);
        else assign_bf16_kernel<4, false><<<grid, threads, 0, s>>>(B);
    }
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

static int launch_assign(hipStream_t s, const float* x, const uint16_t* centers, int64_t rows,
                         int C, int HD, void* ids, int id_bytes) {
    if (rows <= 0) return NKV_OK;
    if (C <= AB_MAXC && HD > 0 && HD % AB_SEG == 0 && HD <= AB_MAXK && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(centers) % 16 == 0) {
        EncBatch B{};
        B.n = 1;
        B.K = HD;
        B.num_centers = C;
        B.id_bytes = id_bytes;
        B.p[0].x = x;
        B.p[0].ldx = HD;
        B.p[0].centers = centers;
        B.p[0].ids = ids;
        B.p[0].M = rows;
        return launch_assign_batch(s, B, false);
    }
    if (HD > 0 && HD % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(centers) % 8 == 0) {
        dim3 grid((unsigned)cdiv(rows, AM_ROWS));
        if (id_bytes == 1)
            assign_mfma_kernel<1><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
        else if (id_bytes == 2)
            assign_mfma_kernel<2><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
        else
            assign_mfma_kernel<4><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
        NKV_LAUNCH_CHECK();
        return NKV_OK;
    }
    dim3 grid((unsigned)cdiv(rows, AS_ROWS));
    if (id_bytes == 1)
        assign_kernel<1><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
    else if (id_bytes == 2)
        assign_kernel<2><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
    else
        assign_kernel<4><<<grid, 256, 0, s>>>(x, centers, rows, C, HD, ids);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

static int check_ids(int C, int id_bytes) {
    NKV_REQUIRE(id_bytes == 1 || id_bytes == 2 || id_bytes == 4, NKV_ERR_INVALID,
                "id_bytes must be 1, 2 or 4");
    NKV_REQUIRE(C > 0, NKV_ERR_INVALID, "need at least one center");
    NKV_REQUIRE(!(id_bytes == 1 && C > 256), NKV_ERR_INVALID, "uint8 ids need C <= 256");
    NKV_REQUIRE(!(id_bytes == 2 && C > 65536), NKV_ERR_INVALID, "uint16 ids need C <= 65536");
    return NKV_OK;
}

namespace {
size_t fit_ws_align(size_t n) { return (n + 255) / 256 * 256; }
}  // namespace

extern "C" size_t nkv_c64_fit_workspace_size(int B, int64_t S, int C) {
    if (B <= 0 || S <= 0 || C <= 0) return 0;
    return 2 * fit_ws_align((size_t)B * C * sizeof(int32_t)) +
           fit_ws_align((size_t)B * S * sizeof(int32_t));
}

extern "C" int nkv_c64_fit(void* stream, const float* x, int B, int64_t S, int HD, int C,
                           int iterations, const int32_t* init_rows, float* centers,
                           int32_t* labels, void* workspace, size_t workspace_bytes) {
    clear_error();
    NKV_REQUIRE(B >= 0 && S >= 0 && HD > 0, NKV_ERR_INVALID, "bad shape");
    NKV_REQUIRE(iterations >= 0, NKV_ERR_INVALID, "iterations must be >= 0");
    if (B == 0 || S == 0) return NKV_OK;
    NKV_REQUIRE(C >= 1 && C <= S && C <= FIT_MAXC, NKV_ERR_INVALID,
                "C64 clusters must be in [1, min(S, 256)]");
    NKV_REQUIRE(S < INT32_MAX, NKV_ERR_INVALID, "rows must fit in 32 bits");
    NKV_REQUIRE(x && init_rows && centers && labels, NKV_ERR_INVALID, "null pointer");
    const size_t need = nkv_c64_fit_workspace_size(B, S, C);
    NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_ERR_WORKSPACE,
                "workspace missing or smaller than nkv_c64_fit_workspace_size()");
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(ws);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + fit_ws_align((size_t)B * C * 4));
    int32_t* order = reinterpret_cast<int32_t*>(ws + 2 * fit_ws_align((size_t)B * C * 4));
    hipStream_t s = (hipStream_t)stream;
    const int64_t elems = (int64_t)B * C * HD;
    c64_init_kernel<<<dim3((unsigned)std::min<int64_t>(cdiv(elems, 256), 4096)), 256, 0, s>>>(
        x, B, S, HD, C, init_rows, centers);
    NKV_LAUNCH_CHECK();
    if (iterations == 0) {
        // no round: the labels stay zero, as the reference initialises them
        zero_i32_kernel<<<dim3((unsigned)std::min<int64_t>(cdiv((int64_t)B * S, 256), 4096)), 256,
                          0, s>>>(labels, (int64_t)B * S);
        NKV_LAUNCH_CHECK();
        return NKV_OK;
    }
    for (int it = 0; it < iterations; ++it) {
        for (int b = 0; b < B; ++b) {
            int rc = launch_assign_f32(s, x + (int64_t)b * S * HD, centers + (int64_t)b * C * HD,
                                       S, C, HD, labels + (int64_t)b * S);
            if (rc) return rc;
        }
        c64_sort_kernel<<<dim3((unsigned)B), FIT_THREADS, 0, s>>>(labels, S, C, counts, offsets,
                                                                  order);
        NKV_LAUNCH_CHECK();
        c64_update_kernel<<<dim3((unsigned)cdiv(HD, 256), (unsigned)C, (unsigned)B), 256, 0, s>>>(
            x, S, HD, C, counts, offsets, order, centers);
        NKV_LAUNCH_CHECK();
    }
    return NKV_OK;
}

extern "C" int nkv_assign(void* stream, const float* x, const uint16_t* centers, int64_t rows,
                          int C, int HD, void* ids, int id_bytes) {
    clear_error();
    NKV_REQUIRE(rows >= 0 && HD > 0, NKV_ERR_INVALID, "rows must be >= 0 and HD > 0");
    int rc = check_ids(C, id_bytes);
    if (rc) return rc;
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(x && centers && ids, NKV_ERR_INVALID, "null pointer");
    return launch_assign((hipStream_t)stream, x, centers, rows, C, HD, ids, id_bytes);
}

namespace {

// Checks of one encode problem; the batch's shape and settings are those of
// its first problem.
int check_encode(const nkv_encode_args* a, const nkv_encode_args* first) {
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null args");
    NKV_REQUIRE(a->rows >= 0, NKV_ERR_INVALID, "rows must be >= 0");
    NKV_REQUIRE(a->HD > 0 && a->HD % 32 == 0, NKV_ERR_INVALID, "HD must be a multiple of 32");
    int rc = check_codec_layout(a->r, a->group, a->scale_dtype);
    if (rc) return rc;
    NKV_REQUIRE(a->quant_mode == NKV_QUANT_FP32 || a->quant_mode == NKV_QUANT_BF16,
                NKV_ERR_INVALID, "bad quant_mode");
    if (a->centers) {
        rc = check_ids(a->num_centers, a->id_bytes);
        if (rc) return rc;
        NKV_REQUIRE(a->ids, NKV_ERR_INVALID, "ids required with centers");
    }
    NKV_REQUIRE(!(a->x && a->x_bf16), NKV_ERR_INVALID, "give x or x_bf16, not both");
    NKV_REQUIRE(a->x_stride == 0 || a->x_stride >= a->HD, NKV_ERR_INVALID,
                "x_stride must be 0 or at least HD");
    if (first != a) {
        NKV_REQUIRE(a->HD == first->HD && a->r == first->r && a->group == first->group &&
                        a->scale_dtype == first->scale_dtype &&
                        a->quant_mode == first->quant_mode &&
                        (a->centers != nullptr) == (first->centers != nullptr) &&
                        a->num_centers == first->num_centers && a->id_bytes == first->id_bytes &&
                        a->ids_in == first->ids_in &&
                        (a->x_bf16 != nullptr) == (first->x_bf16 != nullptr) &&
                        (a->mean != nullptr) == (first->mean != nullptr),
                    NKV_ERR_INVALID,
                    "the problems of one encode batch must share HD, r, group, scale and quant "
                    "settings, center count and id type, and the input dtype");
    }
    if (a->rows == 0) return NKV_OK;
    NKV_REQUIRE((a->x || a->x_bf16) && a->w_enc && a->coeff && a->packed && a->scales,
                NKV_ERR_INVALID, "null pointer");
    return NKV_OK;
}

int encode_batch(hipStream_t s, const nkv_encode_args* a, int n) {
    NKV_REQUIRE(a && n >= 1 && n <= ENC_MAXB, NKV_ERR_INVALID, "1..8 encode problems");
    for (int i = 0; i < n; ++i) {
        int rc = check_encode(a + i, a);
        if (rc) return rc;
    }
    const int HD = a->HD, r = a->r;
    const bool xb = a->x_bf16 != nullptr;
    EncBatch B{};
    B.n = n;
    B.K = HD;
    B.r = r;
    B.num_centers = a->num_centers;
    B.id_bytes = a->id_bytes;
    bool aligned = true;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) {
        const nkv_encode_args& q = a[i];
        EncProb& P = B.p[i];
        P.x = q.x;
        P.xb = q.x_bf16;
        P.ldx = q.x_stride ? q.x_stride : HD;
        P.centers = q.centers;
        P.ids = q.ids;
        P.mean = q.mean;
        P.w_enc = q.w_enc;
        P.coeff = q.coeff;
        P.packed = q.packed;
        P.scales = q.scales;
        P.M = q.rows;
        rows = std::max(rows, q.rows);
        const uintptr_t xp = reinterpret_cast<uintptr_t>(xb ? (const void*)q.x_bf16 : (const void*)q.x);
        aligned = aligned && xp % 16 == 0 && (P.ldx * (xb ? 2 : 4)) % 16 == 0 &&
                  (!q.centers || reinterpret_cast<uintptr_t>(q.centers) % 16 == 0);
    }
    if (rows == 0) return NKV_OK;
    // the batched kernels: the exact bf16-MFMA search (C <= 256) and the
    // staged projection; a bf16 input takes only those
    const bool fast_search = a->num_centers <= AB_MAXC && HD % AB_SEG == 0 && HD <= AB_MAXK;
    const bool fast_proj = HD % 256 == 0;
    static_assert(256 % EP_KS == 0, "the staged projection needs HD % EP_KS == 0");
    const bool search = a->centers && !a->ids_in;
    NKV_REQUIRE(!xb || (aligned && fast_proj && (!search || fast_search)), NKV_ERR_UNSUPPORTED,
                "a bf16 input needs HD % 256 == 0, 16-byte aligned rows and, to search, at most 256 "
                "centers and HD <= 16384");
    int rc = NKV_OK;
    if (search) {
        if (fast_search && aligned) {
            rc = launch_assign_batch(s, B, xb);
        } else {
            for (int i = 0; i < n && !rc; ++i) {
                NKV_REQUIRE(B.p[i].ldx == HD, NKV_ERR_UNSUPPORTED,
                            "a strided fp32 input needs HD % 256 == 0, at most 256 centers and "
                            "16-byte aligned rows");
                rc = launch_assign(s, B.p[i].x, B.p[i].centers, B.p[i].M, B.num_centers, HD,
                                   B.p[i].ids, B.id_bytes);
            }
        }
        if (rc) return rc;
    }
    if (fast_proj && aligned) {
        NKV_REQUIRE(encode_proj_smem() == NKV_OK, NKV_ERR_HIP,
                    "hipFuncSetAttribute failed for the projection kernels");
        B.row_blocks = cdiv(rows, EP_ROWS);
        // groups that do not straddle column blocks are quantised in the same launch
        B.qgroup = EP_COLS % a->group == 0 ? a->group : 0;
        B.scale_dtype = a->scale_dtype;
        B.quant_mode = a->quant_mode;
        const unsigned grid = xcd_grid(n * cdiv(r, EP_COLS) * B.row_blocks);
        if (xb) encode_proj_kernel<true><<<grid, 64 * EP_WAVES, EncProjFmt<true>::SMEM, s>>>(B);
        else encode_proj_kernel<false><<<grid, 64 * EP_WAVES, EncProjFmt<false>::SMEM, s>>>(B);
        NKV_LAUNCH_CHECK();
        if (B.qgroup) return NKV_OK;
    } else {
        for (int i = 0; i < n; ++i) {
            if (B.p[i].M == 0) continue;
            NKV_REQUIRE(B.p[i].ldx == HD, NKV_ERR_UNSUPPORTED,
                        "a strided fp32 input needs HD % 256 == 0 and 16-byte aligned rows");
            EncodeA al;
            al.x = B.p[i].x;
            al.centers = B.p[i].centers;
            al.ids = B.p[i].ids;
            al.id_bytes = B.id_bytes;
            al.num_centers = B.num_centers;
            al.mean = B.p[i].mean;
            al.M = B.p[i].M;
            al.K = HD;
            dim3 grid((unsigned)cdiv(al.M, GT_M), (unsigned)cdiv(r, GT_N));
            encode_gemm_kernel<<<grid, 256, 0, s>>>(al, B.p[i].w_enc, r, B.p[i].coeff);
            NKV_LAUNCH_CHECK();
        }
    }
    const dim3 qgrid((unsigned)cdiv(rows * (r / a->group), 256), (unsigned)n);
    if (a->quant_mode == NKV_QUANT_BF16)
        quant_pack_batch_kernel<NKV_QUANT_BF16><<<qgrid, 256, 0, s>>>(B, a->group, a->scale_dtype);
    else
        quant_pack_batch_kernel<NKV_QUANT_FP32><<<qgrid, 256, 0, s>>>(B, a->group, a->scale_dtype);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

}  // namespace

extern "C" int nkv_encode(void* stream, const nkv_encode_args* a) {
    clear_error();
    return encode_batch((hipStream_t)stream, a, 1);
}

extern "C" int nkv_encode_batch(void* stream, const nkv_encode_args* args, int n) {
    clear_error();
    return encode_batch((hipStream_t)stream, args, n);
}

extern "C" int nkv_decode(void* stream, const nkv_decode_args* a) {
    clear_error();
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null args");
    const nkv_codec& c = a->codec;
    NKV_REQUIRE(a->B >= 1 && a->N >= 0 && a->rows >= 0, NKV_ERR_INVALID, "bad B/N/rows");
    NKV_REQUIRE(a->HD > 0 && a->HD % 32 == 0, NKV_ERR_INVALID, "HD must be a multiple of 32");
    int rc = check_codec_layout(c.r, c.group, c.scale_dtype);
    if (rc) return rc;
    NKV_REQUIRE(a->row_index || a->rows == a->N, NKV_ERR_INVALID,
                "rows must equal N without row_index");
    NKV_REQUIRE(c.n_segments == 0, NKV_ERR_UNSUPPORTED,
                "nkv_decode takes a flat codec; decode segments one at a time");
    if (c.centers) {
        rc = check_ids(c.num_centers, c.id_bytes);
        if (rc) return rc;
        NKV_REQUIRE(c.ids, NKV_ERR_INVALID, "ids required with centers");
    }
    if (a->rows == 0) return NKV_OK;
    NKV_REQUIRE(c.packed && c.scales && c.w_dec && a->out, NKV_ERR_INVALID, "null pointer");
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)cdiv(a->rows, GT_M), (unsigned)cdiv(a->HD, GT_N));
    for (int b = 0; b < a->B; ++b) {
        DecodeA al;
        al.packed = c.packed + (int64_t)b * a->N * (c.r / 2);
        al.scales = c.scales + (int64_t)b * a->N * (c.r / c.group);
        al.row_index = a->row_index;
        al.scale_dtype = c.scale_dtype;
        al.group = c.group;
        al.M = a->rows;
        al.K = c.r;
        DecodeEpi ep;
        ep.centers = c.centers ? c.centers + (int64_t)b * c.centers_batch_stride : nullptr;
        ep.ids = c.ids ? (const void*)((const uint8_t*)c.ids + (int64_t)b * a->N * c.id_bytes)
                       : nullptr;
        ep.id_bytes = c.id_bytes;
        ep.num_centers = c.num_centers;
        ep.row_index = a->row_index;
        ep.mean = c.mean;
        decode_gemm_kernel<<<grid, 256, 0, s>>>(al, ep, c.w_dec, a->HD,
                                                a->out + (int64_t)b * a->rows * a->HD);
        NKV_LAUNCH_CHECK();
    }
    return NKV_OK;
}
