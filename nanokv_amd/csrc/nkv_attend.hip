// nkv_attend.hip -- fused INT4-codec decode + flash attention for gfx950.
//
// One 256-thread block (4 waves, one per SIMD, each with the full 512-entry
// VGPR+AGPR budget) owns one (batch, head) pair, a tile of up to 256 queries
// (64 per wave) and a contiguous range of 32-token key tiles (a "split").
//
// Decoder weights are register-stationary: wave w keeps 64 rows of its
// codec's decoder slice, W[h*128 + 64*(w&1) + [0,64), 0:r) of the K codec
// (waves 0-1) or the V codec (waves 2-3), as MFMA operand fragments for the
// whole kernel (192 registers at r = 384; gfx950 MFMAs read A/B from AGPRs).
// Per history tile p two barrier-separated phases run:
//   A: decode -- K^T = W_K * Z_K^T and V^T = W_V * Z_V^T on MFMA
//      (v_mfma_f32_32x32x16_bf16, fp32 accumulate) from the unpacked codes
//      in LDS, then the reference epilogue bf16(bf16(acc + bf16(mean)) +
//      center[id]) into the bf16 K[token][d] and V^T[d][token] tiles in LDS
//      (the center rows are loaded at the start of the phase, behind the
//      MFMAs);
//   B: attention -- S^T = K * Q^T, P = exp2(S*c - m), O^T += V^T * P^T on
//      MFMA -- with the 16-byte global loads of tile p+1's packed codes
//      issued first and their unpack (code * scale -> bf16) into LDS last.
// Accumulators are kept in VGPRs (-mllvm -amdgpu-mfma-vgpr-form) so the
// softmax and rescale work on them directly; the read-only decoder
// fragments then live in AGPRs.
// Current-chunk tiles (uncompressed bf16) are copied into the K/V tiles
// instead, prefetched a tile ahead.  Decoded K/V never leave LDS.  With more
// than one split the per-split partials (O, m, l) go to the caller's
// workspace and a combine kernel merges them.
//
// MFMA 32x32x16 bf16 operand layout (wave64): lane l supplies row (l % 32)
// of A and column (l % 32) of B with k = 8 * (l / 32) + [0, 8); accumulator
// element i of lane l is (row 8*(i/4) + 4*(l/32) + i%4, column l % 32).
// Keeping queries on the MFMA column axis (S^T, O^T) makes every softmax
// statistic lane-local except one exchange between the two half-waves.
#include "nkv_common.h"
#include "nkv_internal.h"

#include <mutex>
#include <string>

namespace nkv {

constexpr int AT_D = 128;                     // head dim
constexpr int AT_BN = 32;                     // keys per tile
constexpr int AT_THREADS = 256;
constexpr int AT_QB = 2;                      // 32-query blocks per wave
constexpr int AT_BM = 4 * AT_QB * 32;         // at most 256 queries per block
constexpr int AT_RMAX = 384;
constexpr int AT_ZPAD = 8;
constexpr int AT_KPAD = 8;
constexpr int AT_VPAD = 4;
constexpr int AT_ITEMS = 3;  // unpack items per thread: (rK + rV) / 256 <= 3
constexpr int AT_CITEMS = AT_BN * (AT_D / 8) * 2 / AT_THREADS;  // current-tile 16B chunks

struct AttendSmem {
    uint16_t z[2][AT_BN][AT_RMAX + AT_ZPAD];  // unpacked K (0) and V (1) coefficients
    uint16_t ks[AT_BN][AT_D + AT_KPAD];       // K tile [token][d]
    uint16_t vt[AT_D][AT_BN + AT_VPAD];       // V tile, transposed [d][token]
    uint16_t qs[AT_BM][AT_D + AT_KPAD];       // this block's queries [q][d]
    float bias[2][AT_D];
};

struct AttendParams {
    int B, H, S;          // S = splits
    int q_tiles, q_per_tile;
    int64_t Q, N, Nc;
    int t_hist, t_total;  // key tiles (history, all)
    float scale_log2;     // softmax_scale * log2(e)
    int HD;
    const uint16_t* q;
    int64_t q_sb, q_st, q_sh;
    const uint16_t* k_cur;
    int64_t k_sb, k_st, k_sh;
    const uint16_t* v_cur;
    int64_t v_sb, v_st, v_sh;
    nkv_codec codec[2];   // K, V
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    float* ws_o;   // [S, B, H, Q, D]   (S > 1)
    float* ws_ml;  // [S, B, H, Q, 2]
};

// Packed-code streaming.  Thread t owns the work items it = t + 256*e
// (e < AT_ITEMS) of every tile: item it < rK covers 32 K codes (16 bytes,
// one scale) of row it / (rK/32); items rK .. rK+rV-1 cover V.  The item ->
// (codec, row, j) map does not depend on the tile, so it is computed once
// and packed into one register per item; per-codec values are
// kernel-uniform scalars selected per lane (no runtime indexing of the
// argument struct).
struct Streamer {
    const uint8_t* packed0;
    const uint8_t* packed1;
    const uint16_t* scales0;
    const uint16_t* scales1;
    int rowb0, rowb1;    // packed bytes per token (r / 2)
    int ng0, ng1;        // scale groups per token
    int grp0, grp1;      // scale group width
    int fp16_0, fp16_1;  // scale dtype is fp16
    int item[AT_ITEMS];  // row | j << 5 | codec << 9, or -1
};

__device__ __forceinline__ Streamer make_streamer(const nkv_codec& k, const nkv_codec& v,
                                                  const uint8_t* pk, const uint16_t* sk,
                                                  const uint8_t* pv, const uint16_t* sv, int t) {
    Streamer st;
    st.packed0 = pk;
    st.packed1 = pv;
    st.scales0 = sk;
    st.scales1 = sv;
    st.rowb0 = k.r / 2;
    st.rowb1 = v.r / 2;
    st.ng0 = k.r / k.group;
    st.ng1 = v.r / v.group;
    st.grp0 = k.group;
    st.grp1 = v.group;
    st.fp16_0 = k.scale_dtype == NKV_DTYPE_FP16;
    st.fp16_1 = v.scale_dtype == NKV_DTYPE_FP16;
    const int rk = k.r, rv = v.r;
#pragma unroll
    for (int e = 0; e < AT_ITEMS; ++e) {
        int it = t + AT_THREADS * e;
        if (it >= rk + rv) {
            st.item[e] = -1;
        } else if (it < rk) {
            const int row = it / (rk / 32);
            st.item[e] = row | ((it - row * (rk / 32)) << 5);
        } else {
            it -= rk;
            const int row = it / (rv / 32);
            st.item[e] = row | ((it - row * (rv / 32)) << 5) | (1 << 9);
        }
    }
    return st;
}

// Registers carrying one tile from its global loads to its LDS stores.
struct ZPrefetch {
    u32x4 w[AT_ITEMS];  // packed codes
    float s[AT_ITEMS];  // group scales
    int id;             // center id of token l32 in this wave's codec
};

__device__ __forceinline__ void prefetch_tile(ZPrefetch& pf, const Streamer& st,
                                              const void* my_ids, int id_bytes, int ncent,
                                              int64_t tok0, int valid, int t) {
#pragma unroll
    for (int e = 0; e < AT_ITEMS; ++e) {
        const int item = st.item[e];
        const int row = item & 31, j = (item >> 5) & 15, c = (item >> 9) & 1;
        pf.w[e] = u32x4{0, 0, 0, 0};
        pf.s[e] = 0.0f;
        if (item >= 0 && row < valid) {
            const int64_t tok = tok0 + row;
            const uint8_t* src = c ? st.packed1 + tok * st.rowb1 : st.packed0 + tok * st.rowb0;
            pf.w[e] = *reinterpret_cast<const u32x4*>(src + j * 16);
            const uint16_t sb = c ? st.scales1[tok * st.ng1 + (j * 32) / st.grp1]
                                  : st.scales0[tok * st.ng0 + (j * 32) / st.grp0];
            pf.s[e] = (c ? st.fp16_1 : st.fp16_0) ? f16_bits_to_f32(sb) : bf16_bits_to_f32(sb);
        }
    }
    // ids outside the table are clamped so that a corrupt payload cannot read
    // out of bounds (valid payloads never contain them)
    const int tok = t & 31;
    pf.id = (my_ids && tok < valid) ? min(max(read_id(my_ids, id_bytes, tok0 + tok), 0), ncent - 1)
                                    : 0;
}

__device__ __forceinline__ void store_tile(AttendSmem& sm, const ZPrefetch& pf,
                                           const Streamer& st) {
#pragma unroll
    for (int e = 0; e < AT_ITEMS; ++e) {
        const int item = st.item[e];
        if (item < 0) continue;
        const int row = item & 31, j = (item >> 5) & 15, c = (item >> 9) & 1;
        // (nibble - 7) * s = fma(nibble, s, -7 s): both products are exact in
        // fp32 (<= 15 significant bits), so the fma returns the exact value and
        // the bf16 conversion rounds it once, as the reference does.
        const float s = pf.s[e];
        const float ns7 = -7.0f * s;
        u32x4* dst = reinterpret_cast<u32x4*>(&sm.z[c][row][j * 32]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t w = pf.w[e][q];
            const uint32_t ev = w & 0x0f0f0f0fu;          // codes 0, 2, 4, 6 (byte lanes)
            const uint32_t od = (w >> 4) & 0x0f0f0f0fu;   // codes 1, 3, 5, 7
            u32x4 o;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float lo = fmaf((float)((ev >> (8 * b)) & 0xffu), s, ns7);
                const float hi = fmaf((float)((od >> (8 * b)) & 0xffu), s, ns7);
                o[b] = pack_bf16x2(lo, hi);
            }
            dst[q] = o;
        }
    }
}

// Center values the epilogue of this lane adds: token l32 of the tile,
// d = 64*dh + 32*jb + 8*g + 4*hf + [0, 4), as packed bf16 pairs.
__device__ __forceinline__ void load_centers(u32x2 (&cen)[2][4], const uint16_t* centers, int id,
                                             int HD, int h, int dh, int hf) {
    const uint16_t* crow = centers + (int64_t)id * HD + h * AT_D + 64 * dh + 4 * hf;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
            cen[jb][g] = centers ? *reinterpret_cast<const u32x2*>(crow + 32 * jb + 8 * g)
                                 : u32x2{0, 0};
}

// Decode this wave's 64 columns of K (CODEC 0) or V (CODEC 1) for the tile in
// LDS: acc_jb = W[64*dh + 32*jb + .., :] * Z^T (rows d, columns tokens), then
// bf16(bf16(acc + bias) + center) stored as K[token][d] or V^T[d][token].
template <int CODEC, int NKS, int KSMAX>
__device__ __forceinline__ void decode_tile(AttendSmem& sm, const bf16x8 (&wreg)[2][KSMAX],
                                            const u32x2 (&cen)[2][4], bool has_bias, int dh,
                                            int lane) {
    const int hf = lane >> 5, l32 = lane & 31;
    const uint16_t* zrow = &sm.z[CODEC][l32][8 * hf];
    f32x16 acc0 = {}, acc1 = {};
    bf16x8 zn = lds_b128(zrow);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 zf = zn;
        if (ks + 1 < NKS) zn = lds_b128(zrow + 16 * (ks + 1));
        acc0 = mfma32(wreg[0][ks], zf, acc0);
        acc1 = mfma32(wreg[1][ks], zf, acc1);
    }
    const int tok = l32;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 64 * dh + 32 * jb + 8 * g + 4 * hf;
            const f32x16& acc = jb ? acc1 : acc0;
            float a[4] = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
            if (has_bias) {
#pragma unroll
                for (int e = 0; e < 4; ++e) a[e] += sm.bias[CODEC][d + e];
            }
            // first rounding (decoder output), widen, add the bf16 center, round again
            const u32x2 cw = cen[jb][g];
            u32x2 r;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const uint32_t pr = pack_bf16x2(a[2 * h2], a[2 * h2 + 1]);
                const float lo = __uint_as_float(pr << 16) + __uint_as_float(cw[h2] << 16);
                const float hi = __uint_as_float(pr & 0xffff0000u) +
                                 __uint_as_float(cw[h2] & 0xffff0000u);
                r[h2] = pack_bf16x2(lo, hi);
            }
            if (CODEC == 0) {
                *reinterpret_cast<u32x2*>(&sm.ks[tok][d]) = r;
            } else {
                sm.vt[d][tok] = (uint16_t)(r[0] & 0xffffu);
                sm.vt[d + 1][tok] = (uint16_t)(r[0] >> 16);
                sm.vt[d + 2][tok] = (uint16_t)(r[1] & 0xffffu);
                sm.vt[d + 3][tok] = (uint16_t)(r[1] >> 16);
            }
        }
    }
}

// Current-chunk tile chunks: thread t owns 16-byte chunks it = t + 256*e of
// the 32 x 128 K tile (it < 512) and V tile (it >= 512).
struct CurPrefetch {
    u32x4 w[AT_CITEMS];
};

__device__ __forceinline__ void prefetch_current(CurPrefetch& cf, const AttendParams& p, int b,
                                                 int h, int64_t tok0, int valid, int t) {
#pragma unroll
    for (int e = 0; e < AT_CITEMS; ++e) {
        const int it = t + AT_THREADS * e;
        const int kvsel = it / (AT_BN * (AT_D / 8));
        const int rem = it % (AT_BN * (AT_D / 8));
        const int row = rem / (AT_D / 8), d = (rem % (AT_D / 8)) * 8;
        cf.w[e] = u32x4{0, 0, 0, 0};
        if (row < valid) {
            const int64_t tok = tok0 + row;
            const uint16_t* src = kvsel ? p.v_cur + b * p.v_sb + tok * p.v_st + h * p.v_sh + d
                                        : p.k_cur + b * p.k_sb + tok * p.k_st + h * p.k_sh + d;
            cf.w[e] = *reinterpret_cast<const u32x4*>(src);
        }
    }
}

__device__ __forceinline__ void store_current(AttendSmem& sm, const CurPrefetch& cf, int t) {
#pragma unroll
    for (int e = 0; e < AT_CITEMS; ++e) {
        const int it = t + AT_THREADS * e;
        const int kvsel = it / (AT_BN * (AT_D / 8));
        const int rem = it % (AT_BN * (AT_D / 8));
        const int row = rem / (AT_D / 8), d = (rem % (AT_D / 8)) * 8;
        if (!kvsel) {
            *reinterpret_cast<u32x4*>(&sm.ks[row][d]) = cf.w[e];
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sm.vt[d + 2 * q][row] = (uint16_t)(cf.w[e][q] & 0xffffu);
                sm.vt[d + 2 * q + 1][row] = (uint16_t)(cf.w[e][q] >> 16);
            }
        }
    }
}

// One online-softmax step of this wave's two query blocks over the tile in
// LDS.  Blocks past the end of the query tile read zero Q rows; their
// results are never stored.
__device__ __forceinline__ void attend_tile(const AttendSmem& sm, int qrow0,
                                            f32x16 (&o)[AT_QB][AT_D / 32], float (&m_run)[AT_QB],
                                            float (&l_run)[AT_QB], float scale_log2, int valid,
                                            int lane) {
    const int hf = lane >> 5, l32 = lane & 31;
    f32x16 s[AT_QB];
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) s[qb] = f32x16{};
    // S^T = K Q^T: fragments of k-step kk+1 are loaded before the MFMAs of kk
    const uint16_t* krow = &sm.ks[l32][8 * hf];
    const uint16_t* q0row = &sm.qs[qrow0 + l32][8 * hf];
    const uint16_t* q1row = &sm.qs[qrow0 + 32 + l32][8 * hf];
    bf16x8 ka = lds_b128(krow), qa = lds_b128(q0row), qb1 = lds_b128(q1row);
#pragma unroll
    for (int kk = 0; kk < AT_D / 16; ++kk) {
        const bf16x8 a = ka, b0 = qa, b1 = qb1;
        if (kk + 1 < AT_D / 16) {
            ka = lds_b128(krow + 16 * (kk + 1));
            qa = lds_b128(q0row + 16 * (kk + 1));
            qb1 = lds_b128(q1row + 16 * (kk + 1));
        }
        s[0] = mfma32(a, b0, s[0]);
        s[1] = mfma32(a, b1, s[1]);
    }
    bf16x8 pb[AT_QB][2];
    float alpha[AT_QB];
    bool rescale = false;
    if (valid < AT_BN) {  // partial tile: keys past the end get -inf
#pragma unroll
        for (int qb = 0; qb < AT_QB; ++qb)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (8 * (i / 4) + 4 * hf + (i % 4) >= valid) s[qb][i] = -INFINITY;
    }
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) {
        // the max is taken on raw scores (scale_log2 > 0 preserves order)
        float tmax = s[qb][0];
#pragma unroll
        for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[qb][i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32)) * scale_log2;
        const float m_new = fmaxf(m_run[qb], tmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        alpha[qb] = __builtin_amdgcn_exp2f(m_run[qb] - m_use);
        rescale |= m_new > m_run[qb];
        m_run[qb] = m_new;
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // v_exp_f32: exp2 of arguments <= 0; results below 2^-126 flush to 0
            const float e = __builtin_amdgcn_exp2f(fmaf(s[qb][i], scale_log2, -m_use));
            s[qb][i] = e;
            lsum += e;
        }
        l_run[qb] = l_run[qb] * alpha[qb] + lsum;
        // P^T operand of k-step ts: accumulator elements [8*ts, +8), i.e.
        // keys 16*ts + 8*(j/4) + 4*hf + j%4 for slot j
#pragma unroll
        for (int ts = 0; ts < 2; ++ts) {
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = pack_bf16x2(s[qb][8 * ts + 2 * e], s[qb][8 * ts + 2 * e + 1]);
            pb[qb][ts] = as_bf16x8(v);
        }
    }
    // O is rescaled only when some running max of this wave moved (alpha is
    // exactly 1 otherwise); first tiles always move it.
    if (__any(rescale)) {
#pragma unroll
        for (int qb = 0; qb < AT_QB; ++qb)
#pragma unroll
            for (int db = 0; db < AT_D / 32; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[qb][db][i] *= alpha[qb];
    }
    // O^T += V^T P^T: V fragment of step n+1 loaded before the MFMAs of step n
    bf16x8 va = lds_2x64(&sm.vt[l32][4 * hf]);
#pragma unroll
    for (int n = 0; n < 2 * (AT_D / 32); ++n) {
        const int ts = n / (AT_D / 32), db = n % (AT_D / 32);
        const bf16x8 a = va;
        if (n + 1 < 2 * (AT_D / 32)) {
            const int ts1 = (n + 1) / (AT_D / 32), db1 = (n + 1) % (AT_D / 32);
            va = lds_2x64(&sm.vt[32 * db1 + l32][16 * ts1 + 4 * hf]);
        }
        o[0][db] = mfma32(a, pb[0][ts], o[0][db]);
        o[1][db] = mfma32(a, pb[1][ts], o[1][db]);
    }
}

// RK, RV: ranks of the K and V codecs (compile-time, so each decode wave
// runs a branch-free unrolled MFMA chain over its rank).
template <int RK, int RV>
__global__ void __launch_bounds__(AT_THREADS, 1) attend_kernel(AttendParams p) {
    constexpr int KSK = RK / 16, KSV = RV / 16;
    constexpr int KSMAX = KSK > KSV ? KSK : KSV;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    AttendSmem& sm = *reinterpret_cast<AttendSmem*>(smem_raw);

    const int t = threadIdx.x, lane = t & 63;
    // the wave index is uniform; readfirstlane lets the compiler keep every
    // role-dependent value (codec, rank, pointers, loop bounds) in SGPRs and
    // branch on them with scalar branches instead of exec masks
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hf = lane >> 5, l32 = lane & 31;

    // block -> (bh, q tile, split); bh varies fastest so that with B*H a
    // multiple of 8 every block of one head lands on the same XCD (the
    // dispatcher assigns blocks to the 8 XCDs round-robin) and that head's
    // decoder weights stay in one L2.
    const int BH = p.B * p.H;
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int rest = bid / BH;
    const int qt = rest % p.q_tiles;
    const int split = rest / p.q_tiles;
    const int b = bh / p.H, h = bh % p.H;

    const int tile_begin = (int)((int64_t)split * p.t_total / p.S);
    const int tile_end = (int)((int64_t)(split + 1) * p.t_total / p.S);
    const int hist_end = min(tile_end, p.t_hist);

    const nkv_codec& ck = p.codec[0];
    const nkv_codec& cv = p.codec[1];
    const int64_t N = p.N;
    const uint8_t* kpacked = ck.packed ? ck.packed + (int64_t)b * N * (ck.r / 2) : nullptr;
    const uint16_t* kscales = ck.scales ? ck.scales + (int64_t)b * N * (ck.r / ck.group) : nullptr;
    const uint8_t* vpacked = cv.packed ? cv.packed + (int64_t)b * N * (cv.r / 2) : nullptr;
    const uint16_t* vscales = cv.scales ? cv.scales + (int64_t)b * N * (cv.r / cv.group) : nullptr;

    // this wave's decode role: codec (0 = K, 1 = V) and 64-row half dh
    const int codec = wave >> 1, dh = wave & 1;
    const bool has_c = codec ? cv.centers != nullptr : ck.centers != nullptr;
    const uint16_t* my_centers =
        has_c ? (codec ? cv.centers + (int64_t)b * cv.centers_batch_stride
                       : ck.centers + (int64_t)b * ck.centers_batch_stride)
              : nullptr;
    const void* my_ids =
        has_c ? (const void*)((const uint8_t*)(codec ? cv.ids : ck.ids) +
                              (int64_t)b * N * (codec ? cv.id_bytes : ck.id_bytes))
              : nullptr;
    const int my_id_bytes = codec ? cv.id_bytes : ck.id_bytes;
    const int my_ncent = codec ? cv.num_centers : ck.num_centers;
    const int my_r = codec ? cv.r : ck.r;
    const uint16_t* my_wdec = codec ? cv.w_dec : ck.w_dec;
    const bool has_bias = (codec ? cv.mean : ck.mean) != nullptr;

    if (t < AT_D) {
        sm.bias[0][t] = ck.mean ? bf16_round(ck.mean[h * AT_D + t]) : 0.0f;
        sm.bias[1][t] = cv.mean ? bf16_round(cv.mean[h * AT_D + t]) : 0.0f;
    }

    // Q tile -> LDS (rows past the tile end are zero)
    const int64_t tile_q0 = (int64_t)qt * p.q_per_tile;
    const int64_t tile_q1 = min(p.Q, tile_q0 + p.q_per_tile);
    for (int it = t; it < AT_BM * (AT_D / 8); it += AT_THREADS) {
        const int row = it / (AT_D / 8), d = (it % (AT_D / 8)) * 8;
        const int64_t qi = tile_q0 + row;
        u32x4 v = {0, 0, 0, 0};
        if (qi < tile_q1)
            v = *reinterpret_cast<const u32x4*>(p.q + b * p.q_sb + qi * p.q_st + h * p.q_sh + d);
        *reinterpret_cast<u32x4*>(&sm.qs[row][d]) = v;
    }
    const int qrow0 = wave * (AT_QB * 32);
    const int64_t q0 = tile_q0 + qrow0;
    const int nqb = q0 >= tile_q1 ? 0 : (int)min((int64_t)AT_QB, cdiv(tile_q1 - q0, 32));

    // register-stationary decoder fragments: rows 64*dh + 32*jb + l32 of this
    // wave's codec slice, k = 16*ks + 8*hf + [0, 8)
    const bool decodes = hist_end > tile_begin;
    bf16x8 wreg[2][KSMAX];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const uint16_t* wrow =
            my_wdec + (int64_t)(h * AT_D + 64 * dh + 32 * jb + l32) * my_r + 8 * hf;
#pragma unroll
        for (int ks = 0; ks < KSMAX; ++ks) {
            u32x4 v = {0, 0, 0, 0};
            if (decodes && 16 * ks < my_r) v = *reinterpret_cast<const u32x4*>(wrow + 16 * ks);
            wreg[jb][ks] = as_bf16x8(v);
        }
    }

    f32x16 o[AT_QB][AT_D / 32];
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb)
#pragma unroll
        for (int db = 0; db < AT_D / 32; ++db) o[qb][db] = f32x16{};
    float m_run[AT_QB], l_run[AT_QB];
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) {
        m_run[qb] = -INFINITY;
        l_run[qb] = 0.0f;
    }

    auto tile_valid = [&](int tile) {
        return (int)min((int64_t)AT_BN, N - (int64_t)tile * AT_BN);
    };

    // ---- history tiles
    if (tile_begin < hist_end) {
        const Streamer st = make_streamer(ck, cv, kpacked, kscales, vpacked, vscales, t);
        // the center ids of the tile in LDS, for this lane's token (l32)
        int cur_id;
        {
            ZPrefetch pf;
            prefetch_tile(pf, st, my_ids, my_id_bytes, my_ncent, (int64_t)tile_begin * AT_BN,
                          tile_valid(tile_begin), t);
            store_tile(sm, pf, st);
            cur_id = pf.id;
        }
        __syncthreads();  // Q, bias and the first unpacked tile are in LDS
        for (int tile = tile_begin; tile < hist_end; ++tile) {
            // phase A: decode this tile into the K/V tile buffers; the center
            // loads are issued first and land while the decode MFMAs run
            {
                u32x2 cen[2][4];
                load_centers(cen, my_centers, cur_id, p.HD, h, dh, hf);
                if (codec == 0) decode_tile<0, KSK>(sm, wreg, cen, has_bias, dh, lane);
                else decode_tile<1, KSV>(sm, wreg, cen, has_bias, dh, lane);
            }
            __syncthreads();
            // phase B: load the next tile's codes, attend this tile while they
            // arrive, then unpack them into the (now free) coefficient buffers
            ZPrefetch pf;
            const bool next = tile + 1 < hist_end;
            if (next)
                prefetch_tile(pf, st, my_ids, my_id_bytes, my_ncent, (int64_t)(tile + 1) * AT_BN,
                              tile_valid(tile + 1), t);
            attend_tile(sm, qrow0, o, m_run, l_run, p.scale_log2, tile_valid(tile), lane);
            if (next) {
                store_tile(sm, pf, st);
                cur_id = pf.id;
            }
            __syncthreads();
        }
    } else {
        __syncthreads();  // Q and bias are in LDS
    }

    // ---- current-chunk tiles (uncompressed), prefetched a tile ahead
    const int cur_begin = max(tile_begin, p.t_hist);
    if (cur_begin < tile_end) {
        auto cur_valid = [&](int tile) {
            return (int)min((int64_t)AT_BN, p.Nc - (int64_t)(tile - p.t_hist) * AT_BN);
        };
        CurPrefetch cf;
        prefetch_current(cf, p, b, h, (int64_t)(cur_begin - p.t_hist) * AT_BN,
                         cur_valid(cur_begin), t);
        for (int tile = cur_begin; tile < tile_end; ++tile) {
            store_current(sm, cf, t);
            if (tile + 1 < tile_end)
                prefetch_current(cf, p, b, h, (int64_t)(tile + 1 - p.t_hist) * AT_BN,
                                 cur_valid(tile + 1), t);
            __syncthreads();
            attend_tile(sm, qrow0, o, m_run, l_run, p.scale_log2, cur_valid(tile), lane);
            __syncthreads();
        }
    }

    // ---- epilogue
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) {
        if (qb >= nqb) continue;
        const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32);
        const int64_t qi = q0 + 32 * qb + l32;
        if (qi >= tile_q1) continue;
        if (p.S == 1) {
            const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
            uint16_t* orow = p.out + b * p.o_sb + qi * p.o_st + h * p.o_sh;
#pragma unroll
            for (int db = 0; db < AT_D / 32; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * db + 8 * g + 4 * hf;
                    u32x2 pk = {pack_bf16x2(o[qb][db][4 * g] * inv, o[qb][db][4 * g + 1] * inv),
                                pack_bf16x2(o[qb][db][4 * g + 2] * inv, o[qb][db][4 * g + 3] * inv)};
                    *reinterpret_cast<u32x2*>(orow + d) = pk;
                }
            if (p.lse && hf == 0) {
                const float lse2 = l_tot > 0.0f ? m_run[qb] + log2f(l_tot) : -INFINITY;
                p.lse[((int64_t)b * p.H + h) * p.Q + qi] = lse2 * 0.69314718055994531f;
            }
        } else {
            const int64_t row = (((int64_t)split * p.B + b) * p.H + h) * p.Q + qi;
            float* wo = p.ws_o + row * AT_D;
#pragma unroll
            for (int db = 0; db < AT_D / 32; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * db + 8 * g + 4 * hf;
                    f32x4 v = {o[qb][db][4 * g], o[qb][db][4 * g + 1], o[qb][db][4 * g + 2],
                               o[qb][db][4 * g + 3]};
                    *reinterpret_cast<f32x4*>(wo + d) = v;
                }
            if (hf == 0) {
                p.ws_ml[row * 2] = m_run[qb];
                p.ws_ml[row * 2 + 1] = l_tot;
            }
        }
    }
}

// Merge the S split partials of every (b, h, q) row: one thread per 4 d.
__global__ void __launch_bounds__(256) combine_kernel(AttendParams p) {
    const int64_t rows = (int64_t)p.B * p.H * p.Q;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= rows * (AT_D / 4)) return;
    const int64_t row = tid / (AT_D / 4);
    const int d = (int)(tid % (AT_D / 4)) * 4;
    const int64_t qi = row % p.Q;
    const int64_t bhi = row / p.Q;
    const int h = (int)(bhi % p.H), b = (int)(bhi / p.H);
    float M = -INFINITY;
    for (int s = 0; s < p.S; ++s) M = fmaxf(M, p.ws_ml[((int64_t)s * rows + row) * 2]);
    const float Muse = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
    f32x4 acc = {0, 0, 0, 0};
    for (int s = 0; s < p.S; ++s) {
        const int64_t sr = (int64_t)s * rows + row;
        const float w = exp2f(p.ws_ml[sr * 2] - Muse);
        L += p.ws_ml[sr * 2 + 1] * w;
        const f32x4 v = *reinterpret_cast<const f32x4*>(p.ws_o + sr * AT_D + d);
        acc += v * w;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint16_t* orow = p.out + b * p.o_sb + qi * p.o_st + h * p.o_sh + d;
    u32x2 pk = {pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
    *reinterpret_cast<u32x2*>(orow) = pk;
    if (p.lse && d == 0) {
        const float lse2 = L > 0.0f ? M + log2f(L) : -INFINITY;
        p.lse[((int64_t)b * p.H + h) * p.Q + qi] = lse2 * 0.69314718055994531f;
    }
}

// ---- LSE merge of two partitions (CN/core.py:33-42; fast_kernels.py:30-54).
// One wave per row, its lanes striding over d, so that neighbouring lanes
// touch neighbouring elements.  Every lane reads the row's two LSEs before
// lane 0 writes the merged one, so lse_out may alias lse_a or lse_b.
constexpr int LM_WAVES = 4;
__global__ void __launch_bounds__(64 * LM_WAVES) lse_merge_kernel(int64_t rows, int D,
                                                                 const uint16_t* a, int64_t as,
                                                                 const float* la,
                                                                 const uint16_t* bb, int64_t bs,
                                                                 const float* lb, uint16_t* out,
                                                                 int64_t os, float* lo) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * LM_WAVES + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float x = la[row], y = lb[row];
    // logaddexp: max + log1p(exp(-|x - y|)); equal inputs (including -inf) give x + ln 2
    const float l = x == y ? x + 0.69314718055994531f
                           : fmaxf(x, y) + log1pf(expf(-fabsf(x - y)));
    const float origin = isfinite(l) ? l : 0.0f;
    const float wa = expf(x - origin), wb = expf(y - origin);
    for (int d = lane; d < D; d += 64) {
        const float va = bf16_bits_to_f32(a[row * as + d]);
        const float vb = bf16_bits_to_f32(bb[row * bs + d]);
        out[row * os + d] = f32_to_bf16_bits(va * wa + vb * wb);
    }
    if (lo && lane == 0) lo[row] = l;
}

}  // namespace nkv

using namespace nkv;

// ============================================================ C ABI
namespace {

int device_cu_count() {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

struct AttendPlan {
    int q_tiles, q_per_tile, t_hist, t_total, splits;
};

int check_attend_codec(const nkv_codec& c, int64_t N, int HD, const char* which) {
    (void)which;
    NKV_REQUIRE(((c.packed && c.scales) || c.n_segments > 0) && c.w_dec, NKV_ERR_INVALID,
                "history codec needs packed, scales and w_dec");
    NKV_REQUIRE(c.r == 64 || c.r == 128 || c.r == 256 || c.r == 384, NKV_ERR_UNSUPPORTED,
                "fused attend supports codec ranks 64, 128, 256 and 384");
    NKV_REQUIRE(c.group > 0 && c.r % c.group == 0 && c.group % 32 == 0, NKV_ERR_UNSUPPORTED,
                "fused attend needs group to divide r and be a multiple of 32");
    NKV_REQUIRE(c.scale_dtype == NKV_DTYPE_BF16 || c.scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    if (c.centers && c.n_segments == 0) {
        NKV_REQUIRE(c.ids, NKV_ERR_INVALID, "ids required with centers");
        NKV_REQUIRE(c.id_bytes == 1 || c.id_bytes == 2 || c.id_bytes == 4, NKV_ERR_INVALID,
                    "id_bytes must be 1, 2 or 4");
        NKV_REQUIRE(c.num_centers > 0, NKV_ERR_INVALID, "num_centers must be > 0");
    }
    (void)N;
    (void)HD;
    return NKV_OK;
}

int plan_attend(const nkv_attend_args* a, AttendPlan* plan) {
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null args");
    NKV_REQUIRE(a->B >= 1 && a->H >= 1, NKV_ERR_INVALID, "B and H must be >= 1");
    NKV_REQUIRE(a->D == AT_D, NKV_ERR_UNSUPPORTED, "fused attend supports D == 128");
    NKV_REQUIRE(a->Q >= 0 && a->N >= 0 && a->Nc >= 0, NKV_ERR_INVALID, "negative length");
    NKV_REQUIRE(a->splits >= 0, NKV_ERR_INVALID, "splits must be >= 0");
    const int HD = a->H * a->D;
    if (a->N > 0) {
        int rc = check_attend_codec(a->key, a->N, HD, "key");
        if (rc) return rc;
        rc = check_attend_codec(a->value, a->N, HD, "value");
        if (rc) return rc;
    }
    if (a->Nc > 0) NKV_REQUIRE(a->k_cur && a->v_cur, NKV_ERR_INVALID, "current K/V missing");
    if (a->Q > 0) NKV_REQUIRE(a->q && a->out, NKV_ERR_INVALID, "q and out required");
    if (a->Q > 0)
        NKV_REQUIRE(rows16(a->q, a->q_sb, a->q_st, a->q_sh) &&
                        rows16(a->out, a->o_sb, a->o_st, a->o_sh),
                    NKV_ERR_INVALID, "q and out must be 16-byte aligned with strides divisible by 8");
    if (a->Nc > 0)
        NKV_REQUIRE(rows16(a->k_cur, a->k_sb, a->k_st, a->k_sh) &&
                        rows16(a->v_cur, a->v_sb, a->v_st, a->v_sh),
                    NKV_ERR_INVALID,
                    "k_cur and v_cur must be 16-byte aligned with strides divisible by 8");
    plan->q_tiles = (int)cdiv(a->Q, AT_BM);
    // spread the queries evenly over the tiles, in whole 32-query blocks
    plan->q_per_tile =
        plan->q_tiles ? (int)(cdiv(cdiv(a->Q, plan->q_tiles), 32) * 32) : AT_BM;
    plan->t_hist = (int)cdiv(a->N, AT_BN);
    plan->t_total = plan->t_hist + (int)cdiv(a->Nc, AT_BN);
    int S = a->splits;
    const int64_t base = (int64_t)a->B * a->H * plan->q_tiles;
    if (S == 0) {
        // Fill the CUs (one resident block each): minimise waves/S, prefer fewer splits.
        const int cus = device_cu_count();
        double best = 1e30;
        S = 1;
        for (int s = 1; s <= 16 && s <= std::max(1, plan->t_total); ++s) {
            const double waves = (double)cdiv(base * s, cus) / s;
            if (waves < best - 1e-9) {
                best = waves;
                S = s;
            }
        }
    }
    S = std::max(1, std::min(S, std::max(1, plan->t_total)));
    plan->splits = S;
    return NKV_OK;
}

size_t workspace_bytes_for(const nkv_attend_args* a, const AttendPlan& pl) {
    if (pl.splits <= 1) return 0;
    const size_t rows = (size_t)pl.splits * a->B * a->H * a->Q;
    return rows * AT_D * sizeof(float) + rows * 2 * sizeof(float);
}

typedef void (*AttendKernel)(AttendParams);

template <int RK>
AttendKernel attend_instance_rv(int rv) {
    switch (rv) {
        case 64: return attend_kernel<RK, 64>;
        case 128: return attend_kernel<RK, 128>;
        case 256: return attend_kernel<RK, 256>;
        case 384: return attend_kernel<RK, 384>;
        default: return nullptr;
    }
}

AttendKernel attend_instance(int rk, int rv) {
    switch (rk) {
        case 64: return attend_instance_rv<64>(rv);
        case 128: return attend_instance_rv<128>(rv);
        case 256: return attend_instance_rv<256>(rv);
        case 384: return attend_instance_rv<384>(rv);
        default: return nullptr;
    }
}

}  // namespace

namespace {

// Resolve NKV_SCHEDULE_AUTO: key chunks whenever the codecs fit the chunk
// kernels (D = 128, ranks multiples of 64, scale groups multiples of 32),
// query tiles otherwise.  Measured on MI355X at every query count tried,
// 1 .. 320 queries with 2 .. 24 heads and 700 .. 49,920 history keys, the
// key-chunk decomposition (the staged schedule from 8 query blocks) was
// faster: e.g. 0.17 vs 0.24 ms for one query over 12,480 keys at 24 heads,
// 0.60 vs 0.86 ms for 256 queries over 49,920 keys.  Read-time RoPE and the
// other read-time features are built into the key-chunk kernels only.
bool key_chunks_only(const nkv_attend_args* a) {
    return a->rope || a->camera || a->hist_rows || a->cur_mask ||
           (a->N > 0 && (a->key.n_segments > 0 || a->value.n_segments > 0));
}

int resolve_schedule(const nkv_attend_args* a, int* schedule) {
    NKV_REQUIRE(a->schedule >= NKV_SCHEDULE_AUTO && a->schedule <= NKV_SCHEDULE_KEY_CHUNKS,
                NKV_ERR_INVALID, "unknown schedule");
    int sch = a->schedule;
    if (sch == NKV_SCHEDULE_AUTO) {
        const bool fits = a->D == 128 &&
                          (a->N == 0 || (a->key.r % 64 == 0 && a->value.r % 64 == 0 &&
                                         a->key.group % 32 == 0 && a->value.group % 32 == 0));
        sch = fits ? NKV_SCHEDULE_KEY_CHUNKS : NKV_SCHEDULE_QUERY_TILES;
    }
    NKV_REQUIRE(!key_chunks_only(a) || sch == NKV_SCHEDULE_KEY_CHUNKS, NKV_ERR_UNSUPPORTED,
                "read-time RoPE, the camera, history row lists, current-key masks and "
                "segmented codecs need the key-chunk schedule (D = 128, ranks that are "
                "multiples of 64, scale groups that are multiples of 32)");
    *schedule = sch;
    return NKV_OK;
}

}  // namespace

// ------------------------------------------------- heads narrower than 128
// A head width D < 128 (D % 8 == 0; BASELINE config 0 has D = 64) runs
// through the D = 128 kernels on operands padded with zero columns to 128 per
// head.  The zero dimensions add nothing to q.k, and the padded decoder rows,
// centers and mean make every padded history row exactly the decoded row
// followed by zeros (bf16(bf16(0 + 0) + 0) = 0), so the first D columns of
// the output are the attention at width D (the caller's softmax_scale is
// used as given).  The padded q, current K/V, output, decoder weights,
// centers and means sit at the front of the caller's workspace; the rest is
// the D = 128 call's workspace.  RoPE, the camera and segmented codecs keep
// their D = 128 requirement.
namespace {

// [rows = B*T, H, D] strided bf16 -> [rows, H, 128] contiguous, one 16-byte
// unit per thread, zero units past D
__global__ void __launch_bounds__(256) pad_heads_kernel(const uint16_t* __restrict__ src,
                                                        int64_t sb, int64_t st, int64_t sh,
                                                        int64_t T, int H, int D, int64_t rows,
                                                        uint16_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * H * (AT_D / 8)) return;
    const int c = (int)(i % (AT_D / 8));
    const int64_t rh = i / (AT_D / 8);
    const int h = (int)(rh % H);
    const int64_t row = rh / H;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (c < D / 8)
        v = *reinterpret_cast<const u32x4*>(src + (row / T) * sb + (row % T) * st + h * sh + 8 * c);
    *reinterpret_cast<u32x4*>(dst + 8 * i) = v;
}

// the reverse: the first D columns of [rows, H, 128] into the strided output
__global__ void __launch_bounds__(256) unpad_heads_kernel(const uint16_t* __restrict__ src,
                                                          int64_t T, int H, int D, int64_t rows,
                                                          uint16_t* __restrict__ dst, int64_t sb,
                                                          int64_t st, int64_t sh) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int per = D / 8;
    if (i >= rows * H * per) return;
    const int c = (int)(i % per);
    const int64_t rh = i / per;
    const int h = (int)(rh % H);
    const int64_t row = rh / H;
    *reinterpret_cast<u32x4*>(dst + (row / T) * sb + (row % T) * st + h * sh + 8 * c) =
        *reinterpret_cast<const u32x4*>(src + (rh * AT_D + 8 * c));
}

// [A, D, W] -> [A, 128, W] of 16-bit elements, zero rows past D (decoder
// rows [H, D, r], center tables [C*H, D, 1], fp32 means as [H, D, 2])
__global__ void __launch_bounds__(256) pad_rows_kernel(const uint16_t* __restrict__ src, int64_t A,
                                                       int D, int64_t W, uint16_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= A * AT_D * W) return;
    const int64_t w = i % W, rest = i / W;
    const int d = (int)(rest % AT_D);
    const int64_t a = rest / AT_D;
    dst[i] = d < D ? src[(a * D + d) * W + w] : (uint16_t)0;
}

constexpr size_t kNarrowAlign = 256;
inline size_t narrow_round(size_t x) { return (x + kNarrowAlign - 1) & ~(kNarrowAlign - 1); }

// byte offsets of the padded operands in the workspace; inner = the D = 128
// call's workspace start
struct NarrowLayout {
    size_t q, o, kc, vc, w[2], c[2], m[2], inner;
};

int narrow_check(const nkv_attend_args* a) {
    NKV_REQUIRE(a, NKV_ERR_INVALID, "null args");
    NKV_REQUIRE(a->D > 0 && a->D < AT_D && a->D % 8 == 0, NKV_ERR_UNSUPPORTED,
                "fused attend supports D == 128, or D < 128 with D % 8 == 0");
    NKV_REQUIRE(!a->rope && !a->camera, NKV_ERR_UNSUPPORTED,
                "read-time RoPE and the camera need D == 128");
    NKV_REQUIRE(a->N == 0 || (a->key.n_segments == 0 && a->value.n_segments == 0),
                NKV_ERR_UNSUPPORTED, "segmented codecs need D == 128");
    return NKV_OK;
}

int center_tables(const nkv_attend_args* a, const nkv_codec& c) {
    return c.centers_batch_stride ? a->B : 1;
}

NarrowLayout narrow_layout(const nkv_attend_args* a) {
    NarrowLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = narrow_round(off + bytes);
        return o;
    };
    const size_t row = (size_t)a->H * AT_D * sizeof(uint16_t);
    L.q = take((size_t)a->B * a->Q * row);
    L.o = take((size_t)a->B * a->Q * row);
    L.kc = take((size_t)a->B * a->Nc * row);
    L.vc = take((size_t)a->B * a->Nc * row);
    for (int i = 0; i < 2; ++i) {
        const nkv_codec& c = i ? a->value : a->key;
        if (a->N == 0) continue;
        L.w[i] = take(row * c.r);
        if (c.centers) L.c[i] = take((size_t)center_tables(a, c) * c.num_centers * row);
        if (c.mean) L.m[i] = take((size_t)a->H * AT_D * sizeof(float));
    }
    L.inner = off;
    return L;
}

// The D = 128 arguments over the padded operands at base (base may be a
// placeholder when only the workspace size is wanted: nothing is read).
nkv_attend_args narrow_args(const nkv_attend_args* a, const NarrowLayout& L, unsigned char* base) {
    nkv_attend_args n = *a;
    n.D = AT_D;
    const int64_t hd = (int64_t)a->H * AT_D;
    n.q = reinterpret_cast<const uint16_t*>(base + L.q);
    n.q_sb = a->Q * hd, n.q_st = hd, n.q_sh = AT_D;
    n.out = reinterpret_cast<uint16_t*>(base + L.o);
    n.o_sb = a->Q * hd, n.o_st = hd, n.o_sh = AT_D;
    if (a->Nc > 0) {
        n.k_cur = reinterpret_cast<const uint16_t*>(base + L.kc);
        n.v_cur = reinterpret_cast<const uint16_t*>(base + L.vc);
        n.k_sb = n.v_sb = a->Nc * hd;
        n.k_st = n.v_st = hd;
        n.k_sh = n.v_sh = AT_D;
    }
    if (a->N > 0) {
        for (int i = 0; i < 2; ++i) {
            nkv_codec& c = i ? n.value : n.key;
            c.w_dec = reinterpret_cast<const uint16_t*>(base + L.w[i]);
            if (c.centers) {
                c.centers = reinterpret_cast<const uint16_t*>(base + L.c[i]);
                if (c.centers_batch_stride) c.centers_batch_stride = (int64_t)c.num_centers * hd;
            }
            if (c.mean) c.mean = reinterpret_cast<const float*>(base + L.m[i]);
        }
    }
    return n;
}

// a non-null, aligned stand-in base for the size query
unsigned char* narrow_placeholder() { return reinterpret_cast<unsigned char*>((uintptr_t)1 << 12); }

int inner_workspace(const nkv_attend_args* a, size_t* need);

// workspace bytes of a call at any supported D
int attend_need(const nkv_attend_args* a, size_t* need) {
    if (a && a->D != AT_D) {
        int rc = narrow_check(a);
        if (rc) return rc;
        const NarrowLayout L = narrow_layout(a);
        const nkv_attend_args n = narrow_args(a, L, narrow_placeholder());
        size_t inner = 0;
        rc = inner_workspace(&n, &inner);
        if (rc) return rc;
        *need = L.inner + inner;
        return NKV_OK;
    }
    return inner_workspace(a, need);
}

int inner_workspace(const nkv_attend_args* a, size_t* need) {
    AttendPlan pl;
    int rc = plan_attend(a, &pl);
    if (rc) return rc;
    int sch;
    rc = resolve_schedule(a, &sch);
    if (rc) return rc;
    if (sch == NKV_SCHEDULE_KEY_CHUNKS) {
        rc = chunk_check(a);
        if (rc) return rc;
        *need = chunk_workspace_bytes(a);
    } else {
        *need = workspace_bytes_for(a, pl);
    }
    return NKV_OK;
}

int attend_d128(hipStream_t s, const nkv_attend_args* a, void* workspace, size_t workspace_bytes);

int attend_narrow(hipStream_t s, const nkv_attend_args* a, void* workspace, size_t workspace_bytes) {
    int rc = narrow_check(a);
    if (rc) return rc;
    NKV_REQUIRE(a->B >= 1 && a->H >= 1, NKV_ERR_INVALID, "B and H must be >= 1");
    NKV_REQUIRE(a->Q >= 0 && a->N >= 0 && a->Nc >= 0, NKV_ERR_INVALID, "negative length");
    if (a->Q > 0) {
        NKV_REQUIRE(a->q && a->out, NKV_ERR_INVALID, "q and out required");
        NKV_REQUIRE(rows16(a->q, a->q_sb, a->q_st, a->q_sh) &&
                        rows16(a->out, a->o_sb, a->o_st, a->o_sh),
                    NKV_ERR_INVALID, "q and out must be 16-byte aligned with strides divisible by 8");
    }
    if (a->Nc > 0) {
        NKV_REQUIRE(a->k_cur && a->v_cur, NKV_ERR_INVALID, "current K/V missing");
        NKV_REQUIRE(rows16(a->k_cur, a->k_sb, a->k_st, a->k_sh) &&
                        rows16(a->v_cur, a->v_sb, a->v_st, a->v_sh),
                    NKV_ERR_INVALID,
                    "k_cur and v_cur must be 16-byte aligned with strides divisible by 8");
    }
    if (a->N > 0) {
        for (const nkv_codec* c : {&a->key, &a->value}) {
            rc = check_attend_codec(*c, a->N, a->H * a->D, "");
            if (rc) return rc;
        }
    }
    size_t need = 0;
    rc = attend_need(a, &need);
    if (rc) return rc;
    if (a->Q == 0) return NKV_OK;
    NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_ERR_WORKSPACE,
                "workspace missing or smaller than nkv_attend_workspace_size()");
    unsigned char* base = reinterpret_cast<unsigned char*>(workspace);
    const NarrowLayout L = narrow_layout(a);
    const nkv_attend_args n = narrow_args(a, L, base);
    const int D = a->D;
    auto blocks = [](int64_t work) { return dim3((unsigned)cdiv(work, 256)); };
    const int64_t qrows = (int64_t)a->B * a->Q;
    pad_heads_kernel<<<blocks(qrows * a->H * (AT_D / 8)), 256, 0, s>>>(
        a->q, a->q_sb, a->q_st, a->q_sh, a->Q, a->H, D, qrows, const_cast<uint16_t*>(n.q));
    NKV_LAUNCH_CHECK();
    if (a->Nc > 0) {
        const int64_t crows = (int64_t)a->B * a->Nc;
        pad_heads_kernel<<<blocks(crows * a->H * (AT_D / 8)), 256, 0, s>>>(
            a->k_cur, a->k_sb, a->k_st, a->k_sh, a->Nc, a->H, D, crows, const_cast<uint16_t*>(n.k_cur));
        NKV_LAUNCH_CHECK();
        pad_heads_kernel<<<blocks(crows * a->H * (AT_D / 8)), 256, 0, s>>>(
            a->v_cur, a->v_sb, a->v_st, a->v_sh, a->Nc, a->H, D, crows, const_cast<uint16_t*>(n.v_cur));
        NKV_LAUNCH_CHECK();
    }
    if (a->N > 0) {
        for (int i = 0; i < 2; ++i) {
            const nkv_codec& c = i ? a->value : a->key;
            const nkv_codec& cn = i ? n.value : n.key;
            pad_rows_kernel<<<blocks((int64_t)a->H * AT_D * c.r), 256, 0, s>>>(
                c.w_dec, a->H, D, c.r, const_cast<uint16_t*>(cn.w_dec));
            NKV_LAUNCH_CHECK();
            if (c.centers) {
                const int tables = center_tables(a, c);
                const int64_t A = (int64_t)c.num_centers * a->H;
                for (int t = 0; t < tables; ++t) {
                    pad_rows_kernel<<<blocks(A * AT_D), 256, 0, s>>>(
                        c.centers + t * c.centers_batch_stride, A, D, 1,
                        const_cast<uint16_t*>(cn.centers) + (int64_t)t * A * AT_D);
                    NKV_LAUNCH_CHECK();
                }
            }
            if (c.mean) {
                pad_rows_kernel<<<blocks((int64_t)a->H * AT_D * 2), 256, 0, s>>>(
                    reinterpret_cast<const uint16_t*>(c.mean), a->H, D, 2,
                    reinterpret_cast<uint16_t*>(const_cast<float*>(cn.mean)));
                NKV_LAUNCH_CHECK();
            }
        }
    }
    rc = attend_d128(s, &n, base + L.inner, workspace_bytes - L.inner);
    if (rc) return rc;
    unpad_heads_kernel<<<blocks(qrows * a->H * (D / 8)), 256, 0, s>>>(
        n.out, a->Q, a->H, D, qrows, a->out, a->o_sb, a->o_st, a->o_sh);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

}  // namespace

extern "C" size_t nkv_attend_workspace_size(const nkv_attend_args* a) {
    clear_error();
    size_t need = 0;
    return attend_need(a, &need) ? 0 : need;
}

extern "C" int nkv_attend(void* stream, const nkv_attend_args* a, void* workspace,
                          size_t workspace_bytes) {
    clear_error();
    hipStream_t s = (hipStream_t)stream;
    if (a && a->D != AT_D) return attend_narrow(s, a, workspace, workspace_bytes);
    return attend_d128(s, a, workspace, workspace_bytes);
}

namespace {

int attend_d128(hipStream_t s, const nkv_attend_args* a, void* workspace, size_t workspace_bytes) {
    AttendPlan pl;
    int rc = plan_attend(a, &pl);
    if (rc) return rc;
    int sch;
    rc = resolve_schedule(a, &sch);
    if (rc) return rc;
    if (a->Q == 0) return NKV_OK;
    if (sch == NKV_SCHEDULE_KEY_CHUNKS) return chunk_attend_launch(s, a, workspace, workspace_bytes);
    const size_t need = workspace_bytes_for(a, pl);
    NKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), NKV_ERR_WORKSPACE,
                "workspace missing or smaller than nkv_attend_workspace_size()");

    AttendParams p;
    p.B = a->B;
    p.H = a->H;
    p.S = pl.splits;
    p.q_tiles = pl.q_tiles;
    p.q_per_tile = pl.q_per_tile;
    p.Q = a->Q;
    p.N = a->N;
    p.Nc = a->Nc;
    p.t_hist = pl.t_hist;
    p.t_total = pl.t_total;
    p.scale_log2 = a->softmax_scale * 1.4426950408889634f;
    p.HD = a->H * a->D;
    p.q = a->q;
    p.q_sb = a->q_sb;
    p.q_st = a->q_st;
    p.q_sh = a->q_sh;
    p.k_cur = a->k_cur;
    p.k_sb = a->k_sb;
    p.k_st = a->k_st;
    p.k_sh = a->k_sh;
    p.v_cur = a->v_cur;
    p.v_sb = a->v_sb;
    p.v_st = a->v_st;
    p.v_sh = a->v_sh;
    p.codec[0] = a->key;
    p.codec[1] = a->value;
    p.out = a->out;
    p.o_sb = a->o_sb;
    p.o_st = a->o_st;
    p.o_sh = a->o_sh;
    p.lse = a->lse;
    p.ws_o = nullptr;
    p.ws_ml = nullptr;
    if (pl.splits > 1) {
        const size_t rows = (size_t)pl.splits * a->B * a->H * a->Q;
        p.ws_o = reinterpret_cast<float*>(workspace);
        p.ws_ml = p.ws_o + rows * AT_D;
    }
    if (pl.t_total == 0) {
        // no keys at all: out = 0, lse = -inf  (attention_lse, CN/core.py:48-49)
        p.S = 1;
    }
    const size_t smem = sizeof(AttendSmem);
    const int64_t blocks = (int64_t)a->B * a->H * pl.q_tiles * p.S;
    // ranks of the history codecs select the kernel instance (with no history
    // any instance works: the decode path is never entered)
    const int rk = a->N > 0 ? a->key.r : 384, rv = a->N > 0 ? a->value.r : 384;
    auto kernel = attend_instance(rk, rv);
    NKV_REQUIRE(kernel, NKV_ERR_UNSUPPORTED,
                "fused attend supports codec ranks 64, 128, 256 and 384");
    NKV_HIP_CHECK(hipFuncSetAttribute((const void*)kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    if (a->ev_kernel_begin) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)a->ev_kernel_begin, s));
    kernel<<<dim3((unsigned)blocks), AT_THREADS, smem, s>>>(p);
    NKV_LAUNCH_CHECK();
    if (a->ev_kernel_end) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)a->ev_kernel_end, s));
    if (p.S > 1) {
        const int64_t threads = (int64_t)a->B * a->H * a->Q * (AT_D / 4);
        combine_kernel<<<dim3((unsigned)cdiv(threads, 256)), 256, 0, s>>>(p);
        NKV_LAUNCH_CHECK();
    }
    return NKV_OK;
}

}  // namespace

// ------------------------------------------------- allocation-free nkv_attend
// The scratch of nkv_attend_static: one array per GPU in the code object, so
// a call allocates nothing.  In host code the name `scratch` is only a
// host-side stand-in for the symbol; the device address of each GPU's copy
// comes from hipGetSymbolAddress, once per device (with that device current),
// and only that address is passed to kernels.
static __device__ __align__(256) unsigned char scratch[NKV_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::once_flag g_scratch_once[kScratchDevices];
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_err[kScratchDevices];

// The scratch address of device `dev` (which must be current).
int scratch_address(int dev, void** ptr) {
    NKV_REQUIRE(dev >= 0 && dev < kScratchDevices, NKV_ERR_UNSUPPORTED,
                "device index beyond the static scratch table");
    std::call_once(g_scratch_once[dev], [dev]() {
        void* p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = p;
    });
    if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev]) {
        set_error(std::string("nkv_attend_static: hipGetSymbolAddress failed: ") +
                  hipGetErrorString(g_scratch_err[dev]));
        return NKV_ERR_HIP;
    }
    *ptr = g_scratch_ptr[dev];
    return NKV_OK;
}

}  // namespace

extern "C" int nkv_attend_static(void* stream, const nkv_attend_args* a) {
    clear_error();
    size_t need = 0;
    int rc = attend_need(a, &need);
    if (rc) return rc;
    NKV_REQUIRE(need <= (size_t)NKV_STATIC_SCRATCH_BYTES, NKV_ERR_WORKSPACE,
                "the call needs " + std::to_string(need) + " bytes of scratch; "
                "nkv_attend_static holds " + std::to_string((size_t)NKV_STATIC_SCRATCH_BYTES) +
                " (use nkv_attend with a caller workspace)");
    int dev = 0;
    NKV_HIP_CHECK(hipGetDevice(&dev));
    if (stream) {
        hipDevice_t sdev = 0;
        NKV_HIP_CHECK(hipStreamGetDevice((hipStream_t)stream, &sdev));
        NKV_REQUIRE((int)sdev == dev, NKV_ERR_INVALID,
                    "nkv_attend_static: the stream belongs to another device than the current one");
    }
    void* ptr = nullptr;
    rc = scratch_address(dev, &ptr);
    if (rc) return rc;
    return nkv_attend(stream, a, need ? ptr : nullptr, need);
}

extern "C" int nkv_lse_merge(void* stream, int64_t rows, int D, const uint16_t* a,
                             int64_t a_stride, const float* lse_a, const uint16_t* b,
                             int64_t b_stride, const float* lse_b, uint16_t* out,
                             int64_t out_stride, float* lse_out) {
    clear_error();
    NKV_REQUIRE(rows >= 0 && D > 0, NKV_ERR_INVALID, "rows must be >= 0 and D > 0");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(a && b && lse_a && lse_b && out, NKV_ERR_INVALID, "null pointer");
    lse_merge_kernel<<<dim3((unsigned)cdiv(rows, LM_WAVES)), 64 * LM_WAVES, 0, (hipStream_t)stream>>>(
        rows, D, a, a_stride, lse_a, b, b_stride, lse_b, out, out_stride, lse_out);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
