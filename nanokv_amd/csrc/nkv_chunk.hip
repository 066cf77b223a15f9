// nkv_chunk.hip -- key-chunk-major fused decode + attention for gfx950
// (NKV_SCHEDULE_KEY_CHUNKS of nkv_attend).
//
// A 256-thread block (4 waves, one per SIMD) owns one (batch, head, chunk)
// of 256 keys.  It decodes the chunk's K and V once into LDS -- K[key][d]
// and V^T[d][key], bf16, 136 KB -- and then every wave attends its share of
// ALL query tiles (64 queries each) to those keys.  Each (query, chunk)
// leaves a partial: the chunk-local softmax output O / l as bf16 and its
// log2-sum-exp m + log2(l) as fp32.  A combine kernel merges the partials of
// every query by log-sum-exp (CN/core.py:33-42 applied over all chunks).  A
// 32-query block's partial is stored in the MFMA accumulator's lane order
// (8 KB: eight 1 KB rows of 16 bytes per lane), so the stores here and the
// combine's loads are contiguous.
// Decoding each history key once per head, instead of once per query tile,
// removes the decode GEMM's re-execution; the price is the partial traffic
// (256 + 4 bytes per query and chunk).
//
// Decode (per wave: 64 keys of the chunk, both codecs; MFMA 32x32x16 bf16):
//   K^T = W_K[h*128 + d, :] . Z^T   (A = decoder rows, B = unpacked codes)
//   V   = Z . W_V[h*128 + d, :]^T   (A = unpacked codes, B = decoder rows)
// The k (rank) axis is walked in blocks of 64: lane half hf supplies
// k = 64*kq + 32*hf + 8*j + [0, 8) at step j of block kq.  That permutation of
// the summation index is applied to both operands, so one 16-byte load per
// lane fetches the packed codes of four MFMA steps, and they share one scale
// group (group % 32 == 0).  Decoder rows come straight from global memory
// (L2-resident per head).  The epilogue is the reference decode arithmetic
// bf16(bf16(acc + bf16(mean)) + center[id]) (MG:438-454); the accumulator
// orientation puts four consecutive d (K) or four consecutive keys (V) in
// one lane, so both tiles are written with 8-byte LDS stores.
// Current-chunk keys (uncompressed bf16) are copied instead of decoded.
//
// Attention (per wave and 64-query tile; queries on the MFMA column axis):
//   S^T = K Q^T, P = exp2(S * c - m), O^T += V^T P^T
// over eight 32-key steps, software-pipelined: step j's softmax (VALU) runs
// between the MFMAs of step j+1's scores and step j-1's PV product, which
// do not depend on it.  The running max is raised only when a score exceeds
// it by more than 2^8 (P <= 256 otherwise), so O is rarely rescaled.
#include "nkv_common.h"
#include "nkv_internal.h"

namespace nkv {

#ifdef NKV_PLAIN_STORES
#define NT_STORE(v, ptr) (*(ptr) = (v))
#else
#define NT_STORE(v, ptr) __builtin_nontemporal_store((v), (ptr))
#endif

constexpr int CK_T = 256;        // keys per chunk
constexpr int CK_D = 128;        // head dim
constexpr int CK_THREADS = 256;  // 4 waves
constexpr int CK_KROW = CK_D + 8;   // K row: 68 dwords (b128 reads conflict-free)
constexpr int CK_VROW = CK_T + 4;   // V^T row: 130 dwords (b64 reads conflict-free)
constexpr int CK_QT = 64;        // queries per wave tile
constexpr float CK_TAU = 8.0f;   // lazy-rescale threshold (log2 units)

struct ChunkSmem {
    // K tile [key][DK + 8] (for DK < 128 only the front of the region is the
    // tile); also decoder-slice and center staging during the decode
    uint16_t k[CK_T][CK_KROW];
    uint16_t vt[CK_D][CK_VROW];   // V^T[d][key]
    int ids[2][CK_T];             // center ids of the chunk's keys (K, V)
    float bias[2][CK_D];          // bf16 bias of this head (K, V)
};

// K tile row pitch for a K/Q width DK (b128 reads of 8 rows hit distinct banks)
template <int DK>
struct KTile {
    static constexpr int ROW = DK + 8;
};

struct ChunkParams {
    int B, H;           // H: heads of this launch (launch head i)
    int nch_hist, nch_total;
    int qblocks;        // 32-query blocks per (b, i): cdiv(Q, 32)
    int64_t Q;
    int64_t N;          // history tokens per batch item in the codec arrays
    int64_t n_rows;     // history keys attended
    const int32_t* rows;  // [n_rows] codec rows of those keys, or null: rows 0 .. n_rows-1
    int64_t Nc;
    float scale_log2;
    const uint16_t* q;  // [B, Q, H, DK] (strides)
    int64_t q_sb, q_st, q_sh;
    const uint16_t* k_cur;
    int64_t k_sb, k_st, k_sh;
    const uint16_t* v_cur;
    int64_t v_sb, v_st, v_sh;
    ChunkCodec codec[2];
    uint16_t* part_o;   // [B*H, nch_total, qblocks, 8, 64 lanes, 8] bf16 (lane order)
    float* part_lse;    // [B*H, nch_total, qblocks * 32] log2 domain
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
};

// Codec row of attended history key `key`; rows outside the codec are
// clamped so that a bad row list cannot read out of bounds.
__device__ __forceinline__ int64_t history_row(const ChunkParams& p, int64_t key) {
    if (!p.rows) return key;
    return min(max((int64_t)p.rows[key], (int64_t)0), p.N - 1);
}

// ------------------------------------------------------------------ decode
// This wave's 64 keys (64*wave + [0, 64) of the chunk) of codec CODEC.
// Decoder-slice staging: the block copies W[h*128 + d][64*kq, +64) (16 KB)
// into LDS with coalesced 16-byte loads (8 threads per 128-byte row), double
// buffered, so each decoder element is fetched from L2 once per block and
// every wave reads its MFMA fragments from LDS.  Rows are padded to 72 bf16
// (36 dwords): the b128 fragment reads of 8 consecutive rows hit distinct
// banks.
constexpr int WS_ROW = 72;
constexpr int WS_BUF = CK_D * WS_ROW;  // bf16 elements per buffer
static_assert(2 * WS_BUF <= CK_D * CK_VROW && 2 * WS_BUF <= CK_T * CK_KROW,
              "decoder staging must fit in the V^T and K regions");

// The 128 center values of launch head h for the wave's 64 keys (V),
// with coalesced 16-byte loads (one 256-byte row per 16 lanes) ...
__device__ __forceinline__ void load_center_rows(u32x4 (&v)[16], const ChunkSmem& sm,
                                                 const ChunkCodec& c, int codec, int b, int h,
                                                 int wave, int lane) {
    const uint16_t* cent = c.centers + (int64_t)b * c.c_bs + (int64_t)h * c.c_hs;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int t = 64 * wave + 4 * e + (lane >> 4);
        v[e] = *reinterpret_cast<const u32x4*>(cent + (int64_t)sm.ids[codec][t] * c.c_rs +
                                               8 * (lane & 15));
    }
}

// ... stored into the wave's own K rows of LDS (other waves' rows are not
// touched).
__device__ __forceinline__ void store_center_rows(const u32x4 (&v)[16], ChunkSmem& sm, int wave,
                                                  int lane) {
#pragma unroll
    for (int e = 0; e < 16; ++e)
        *reinterpret_cast<u32x4*>(&sm.k[64 * wave + 4 * e + (lane >> 4)][8 * (lane & 15)]) = v[e];
}

// K center values in the K^T accumulator layout: key 64*wave + 32*tt + l32,
// d = 32*dt + 8*g + 4*hf + [0, 4), dt < NDT.
template <int NDT>
__device__ __forceinline__ void load_k_centers(u32x2 (&cen)[2][NDT][4], const ChunkSmem& sm,
                                               const ChunkCodec& c, int b, int h, int wave,
                                               int lane) {
    const int hf = lane >> 5, l32 = lane & 31;
    const uint16_t* cent = c.centers + (int64_t)b * c.c_bs + (int64_t)h * c.c_hs + 4 * hf;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const uint16_t* crow = cent + (int64_t)sm.ids[0][64 * wave + 32 * tt + l32] * c.c_rs;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                cen[tt][dt][g] = *reinterpret_cast<const u32x2*>(crow + 32 * dt + 8 * g);
    }
}

// Decode this wave's 64 keys of codec CODEC to WIDTH columns (V: 128; K:
// the launch's DK, written to the K tile with row pitch KROW).  wst: 2 *
// WS_BUF bf16 of LDS that no other data uses during the call.  HAS_C: the
// codec has centers (a template argument so that the epilogue is
// straight-line code); V's are staged in the wave's K-region rows, K's are
// loaded during the last slice.  Ends with a block barrier after the last
// read of wst.
template <int CODEC, bool HAS_C, int WIDTH, int KROW>
__device__ __forceinline__ void decode_codec(ChunkSmem& sm, uint16_t* wst, const ChunkCodec& c,
                                             const ChunkParams& p, int b, int h, int64_t tok0,
                                             int valid, int wave, int lane) {
    constexpr int NDT = WIDTH / 32;
    const int hf = lane >> 5, l32 = lane & 31;
    const int R = c.r, KQ = R >> 6, G = c.group, NG = R / G;
    const bool f16 = c.scale_dtype == NKV_DTYPE_FP16;
    const uint8_t* prow[2];
    const uint16_t* srow[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int tl = 64 * wave + 32 * tt + l32;
        // keys past the chunk end decode key 0's codes (finite, never attended)
        const int64_t key = tok0 + (tl < valid ? tl : 0);
        const int64_t tok = (int64_t)b * p.N + history_row(p, key);
        prow[tt] = c.packed + tok * (R / 2) + 16 * hf;
        srow[tt] = c.scales + tok * NG;
    }
    const int t = 64 * wave + lane;
    const uint16_t* wsrc = c.w + (int64_t)h * c.w_hs + (int64_t)(t >> 3) * R + 8 * (t & 7);
    uint16_t* wdst = wst + (t >> 3) * WS_ROW + 8 * (t & 7);
    auto wload = [&](int kq, u32x4 (&r)[NDT]) {
#pragma unroll
        for (int e = 0; e < NDT; ++e)
            r[e] = *reinterpret_cast<const u32x4*>(wsrc + (int64_t)32 * e * R + 64 * kq);
    };
    auto wstore = [&](int buf, const u32x4 (&r)[NDT]) {
#pragma unroll
        for (int e = 0; e < NDT; ++e)
            *reinterpret_cast<u32x4*>(wdst + buf * WS_BUF + 32 * e * WS_ROW) = r[e];
    };
    auto cload = [&](int kq, u32x4 (&pk)[2], float (&sc)[2]) {
        const int gi = (64 * kq + 32 * hf) / G;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            pk[tt] = *reinterpret_cast<const u32x4*>(prow[tt] + 32 * kq);
            const uint16_t sb = srow[tt][gi];
            sc[tt] = f16 ? f16_bits_to_f32(sb) : bf16_bits_to_f32(sb);
        }
    };

    f32x16 acc[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[dt][tt] = f32x16{};

    // V: this wave's center rows go to its own K rows (store_center_rows);
    // their loads are issued first so that they overlap the prologue.
    u32x4 cst[16];
    if (CODEC == 1 && HAS_C) load_center_rows(cst, sm, c, 1, b, h, wave, lane);

    // One slice ahead: codes (HBM) and decoder rows for slice kq+1 are
    // requested while slice kq is multiplied; the rows go to the other LDS
    // buffer at the end of the iteration.
    u32x4 wr[NDT], pk[2];
    float sc[2];
    wload(0, wr);
    cload(0, pk, sc);
    if (CODEC == 1 && HAS_C) store_center_rows(cst, sm, wave, lane);
    wstore(0, wr);
    __syncthreads();
    // fragment rows 32*dt + l32, k = 32*hf + 8*j within the slice
    const uint16_t* wfrag = wst + l32 * WS_ROW + 32 * hf;
    u32x2 cen[2][NDT][4];  // K epilogue center values, requested during the last slice
    for (int kq = 0; kq < KQ; ++kq) {
        u32x4 pkn[2];
        float scn[2];
        const bool more = kq + 1 < KQ;
        if (more) {
            wload(kq + 1, wr);
            cload(kq + 1, pkn, scn);
        }
        if (CODEC == 0 && HAS_C && !more) load_k_centers<NDT>(cen, sm, c, b, h, wave, lane);
        const uint16_t* wb = wfrag + (kq & 1) * WS_BUF;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 z[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) z[tt] = unpack8(pk[tt][j], sc[tt], -7.0f * sc[tt]);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const bf16x8 w = lds_b128(wb + 32 * dt * WS_ROW + 8 * j);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
                    acc[dt][tt] = CODEC == 0 ? mfma32(w, z[tt], acc[dt][tt])
                                             : mfma32(z[tt], w, acc[dt][tt]);
            }
        }
        if (more) {
            // the other buffer was last read before the previous barrier
            wstore((kq + 1) & 1, wr);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                pk[tt] = pkn[tt];
                sc[tt] = scn[tt];
            }
        }
        __syncthreads();
    }

    // Epilogue.  sm.bias holds bf16(mean) or zeros, so the bias add is
    // unconditional.
    if (CODEC == 0) {
        // acc[dt][tt] element i: d = 32*dt + 8*(i/4) + 4*hf + i%4, key
        // 64*wave + 32*tt + l32; cen holds the center values (4 consecutive d
        // per group).
        uint16_t* ktile = &sm.k[0][0];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 64 * wave + 32 * tt + l32;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * dt + 8 * g + 4 * hf;
                    u32x2* slot = reinterpret_cast<u32x2*>(ktile + t * KROW + d);
                    float a[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) a[e] = acc[dt][tt][4 * g + e] + sm.bias[0][d + e];
                    const u32x2 cw = HAS_C ? cen[tt][dt][g] : u32x2{0, 0};
                    u32x2 r;
#pragma unroll
                    for (int h2 = 0; h2 < 2; ++h2) {
                        const uint32_t pr = pack_bf16x2(a[2 * h2], a[2 * h2 + 1]);
                        r[h2] = pack_bf16x2(
                            __uint_as_float(pr << 16) + __uint_as_float(cw[h2] << 16),
                            __uint_as_float(pr & 0xffff0000u) +
                                __uint_as_float(cw[h2] & 0xffff0000u));
                    }
                    *slot = r;
                }
        }
    } else {
        // acc[dt][tt] element i: key 64*wave + 32*tt + 8*(i/4) + 4*hf + i%4, d = 32*dt + l32;
        // the center rows of the wave's keys were staged into its K rows
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int t0 = 64 * wave + 32 * tt + 8 * g + 4 * hf;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const int d = 32 * dt + l32;
                    const float bias = sm.bias[1][d];
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float a = bf16_round(acc[dt][tt][4 * g + e] + bias);
                        v[e] = HAS_C ? a + bf16_bits_to_f32(sm.k[t0 + e][d]) : a;
                    }
                    const u32x2 r = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    *reinterpret_cast<u32x2*>(&sm.vt[d][t0]) = r;
                }
            }
    }
}

// Current-chunk keys: copy K rows, transpose V into V^T (rows past the end
// are zero).
// (Current keys are native: the launch's DK is 128.)
__device__ __forceinline__ void load_current_chunk(ChunkSmem& sm, const ChunkParams& p, int b,
                                                   int h, int64_t tok0, int valid, int t) {
    const bool ok = t < valid;
    const uint16_t* ks = p.k_cur + (int64_t)b * p.k_sb + (tok0 + (ok ? t : 0)) * p.k_st +
                         (int64_t)h * p.k_sh;
    const uint16_t* vs = p.v_cur + (int64_t)b * p.v_sb + (tok0 + (ok ? t : 0)) * p.v_st +
                         (int64_t)h * p.v_sh;
#pragma unroll 4
    for (int e = 0; e < CK_D / 8; ++e) {
        u32x4 kv = *reinterpret_cast<const u32x4*>(ks + 8 * e);
        u32x4 vv = *reinterpret_cast<const u32x4*>(vs + 8 * e);
        if (!ok) kv = vv = u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x4*>(&sm.k[t][8 * e]) = kv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sm.vt[8 * e + 2 * i][t] = (uint16_t)(vv[i] & 0xffffu);
            sm.vt[8 * e + 2 * i + 1][t] = (uint16_t)(vv[i] >> 16);
        }
    }
}

// --------------------------------------------------------------- attention
// The d walk of the score product S^T = K Q^T over a K/Q width DK: at
// k-step kk lane half hf supplies d = dwalk_block(kk) + dwalk_half * hf +
// [0, 8).  The d axis is cut into blocks of 2 * HALF (HALF = min(DK, 64) / 2)
// and each lane half walks 16-byte runs of its half-block, so a lane's
// fragments of consecutive steps are contiguous.  K reads and Q loads use
// the same walk.
template <int DK>
struct DWalk {
    static constexpr int HALF = (DK < 64 ? DK : 64) / 2;
    static constexpr int PER = HALF / 8;  // k-steps per half-block
    static constexpr int KSTEPS = DK / 16;
    static constexpr int block(int kk) { return (kk / PER) * 2 * HALF + 8 * (kk % PER); }
};

// Q^T operand fragments of 32 queries [q_blk, q_blk + 32) (width DK); rows
// past the last query read row q_safe (finite, never stored).
template <int DK>
__device__ __forceinline__ void load_q_block(bf16x8 (&qf)[8], const ChunkParams& p, int b, int h,
                                             int64_t q_blk, int64_t q_safe, int lane) {
    using W = DWalk<DK>;
    const int hf = lane >> 5, l32 = lane & 31;
    const int64_t qi = q_blk + l32;
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (qi < p.Q ? qi : q_safe) * p.q_st +
                           (int64_t)h * p.q_sh + W::HALF * hf;
#pragma unroll
    for (int kk = 0; kk < W::KSTEPS; ++kk)
        qf[kk] = as_bf16x8(*reinterpret_cast<const u32x4*>(qrow + W::block(kk)));
}

// One wave attends queries [q0, q0 + 32*NQB) to the chunk in LDS.  FULL: the
// chunk has all 256 keys (eight pipelined steps); otherwise nsub steps with
// the last one masked to `valid` keys.  qf holds this tile's query
// fragments on entry; as soon as a query block's last score product is
// issued, its registers are refilled with the wave's next tile (first query
// q_next), so that tile's loads overlap this tile's remaining work.
template <int DK, int NQB, bool FULL>
__device__ __forceinline__ void attend_qtile(const ChunkSmem& sm, const ChunkParams& p, int b,
                                             int h, int bh, int chunk, int64_t q0, int nsub,
                                             int valid, int lane_in, bf16x8 (&qf)[2][8],
                                             int64_t q_next) {
    // Opaque per-tile copy of the lane index: every lane-dependent address
    // below is recomputed per tile instead of being hoisted out of the
    // query-tile loop (where it would be spilled: the loop body needs
    // nearly all 256 VGPRs).
    int lane = lane_in;
    asm volatile("" : "+v"(lane));
    const int hf = lane >> 5, l32 = lane & 31;
    const float c = p.scale_log2;

    f32x16 o[NQB][4];
    float m[NQB], l[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        m[qb] = -INFINITY;
        l[qb] = 0.0f;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[qb][db] = f32x16{};
    }

    // K fragments of step j (shared by both query blocks)
    // Fragment addresses are an opaque per-tile base plus compile-time
    // offsets (< 64 KiB, folded into the ds_read instructions); without the
    // opaque step the compiler hoists one address register per unrolled
    // fragment out of the query-tile loop and spills.
    using W = DWalk<DK>;
    constexpr int KROW = KTile<DK>::ROW;
    constexpr int KS = W::KSTEPS;
    uint32_t koff = l32 * KROW + W::HALF * hf, voff = l32 * CK_VROW + 4 * hf;
    asm volatile("" : "+v"(koff));
    asm volatile("" : "+v"(voff));
    const uint16_t* kbase = &sm.k[0][0] + koff;
    const uint16_t* vbase = &sm.vt[0][0] + voff;
    auto load_k = [&](int j, bf16x8 (&kf)[KS]) {
        const uint16_t* kr = kbase + 32 * j * KROW;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kf[kk] = lds_b128(kr + W::block(kk));
    };
    // V^T fragments of step j: P^T operand slot jj of half-step ts holds key
    // 16*ts + 8*(jj/4) + 4*hf + jj%4 (accumulator element 8*ts + jj of S^T),
    // and V^T is read with the same key permutation.
    auto load_v = [&](int j, bf16x8 (&vf)[2][4]) {
#pragma unroll
        for (int ts = 0; ts < 2; ++ts)
#pragma unroll
            for (int db = 0; db < 4; ++db)
                vf[ts][db] = lds_2x64(vbase + 32 * db * CK_VROW + 32 * j + 16 * ts);
    };
    auto qk = [&](int qb, const bf16x8 (&kf)[KS], f32x16& s) {
        s = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) s = mfma32(kf[kk], qf[qb][kk], s);
    };
    auto pv = [&](int qb, const bf16x8 (&vf)[2][4], const bf16x8 (&pb)[2]) {
#pragma unroll
        for (int ts = 0; ts < 2; ++ts)
#pragma unroll
            for (int db = 0; db < 4; ++db) o[qb][db] = mfma32(vf[ts][db], pb[ts], o[qb][db]);
    };
    // online softmax of one 32-key x 32-query score tile; returns whether
    // this lane raised its running max (then O must be scaled by alpha)
    auto softmax = [&](int qb, f32x16& s, bf16x8 (&pb)[2], float& alpha) {
        float tmax = fmaxf(s[0], s[1]);
#pragma unroll
        for (int i = 2; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
        // the max is taken on raw scores (c > 0 preserves order)
        tmax = halfwave_max(tmax) * c;
        const bool up = tmax > m[qb] + CK_TAU;
        const float m_new = up ? tmax : m[qb];
        alpha = up ? __builtin_amdgcn_exp2f(m[qb] - m_new) : 1.0f;
        m[qb] = m_new;
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // v_exp_f32 of arguments <= 8; results below 2^-126 flush to 0
            const float e = __builtin_amdgcn_exp2f(fmaf(s[i], c, -m_new));
            s[i] = e;
            lsum += e;
        }
        l[qb] = l[qb] * alpha + lsum;
        // materialise the row sum here: left alone, the compiler defers these
        // adds to the end of the tile and keeps every exp value alive (spills)
        asm volatile("" : "+v"(l[qb]));
#pragma unroll
        for (int ts = 0; ts < 2; ++ts) {
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = pack_bf16x2(s[8 * ts + 2 * e], s[8 * ts + 2 * e + 1]);
            pb[ts] = as_bf16x8(v);
        }
        return up;
    };
    auto rescale = [&](int qb, float alpha) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[qb][db][i] *= alpha;
    };

    constexpr int NSTEP = CK_T / 32;
    if (FULL && NQB == 2) {
        // Two query blocks staggered by half a step: block 0's softmax runs
        // under block 1's MFMAs and vice versa.  Per step j:
        //   X: S1 = QK(j), O1 += PV(j-1)      | softmax(S0 of step j)
        //   Y: S0 = QK(j+1), O0 += PV(j)      | softmax(S1 of step j)
        f32x16 s0, s1;
        bf16x8 p0[2], p1[2];
        bf16x8 kf[KS], vprev[2][4];
        float a0, a1;
        load_k(0, kf);
        qk(0, kf, s0);
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
            bf16x8 vf[2][4], kn[KS];
            qk(NQB - 1, kf, s1);
            if (j == NSTEP - 1) load_q_block<DK>(qf[1], p, b, h, q_next + 32, q_next, lane);
            if (j > 0) pv(NQB - 1, vprev, p1);
            load_v(j, vf);
            if (j + 1 < NSTEP) load_k(j + 1, kn);
            const bool up0 = softmax(0, s0, p0, a0);
            if (j > 0 && __any(up0)) rescale(0, a0);
            if (j + 1 < NSTEP) qk(0, kn, s0);
            if (j == NSTEP - 2) load_q_block<DK>(qf[0], p, b, h, q_next, q_next, lane);
            pv(0, vf, p0);
            const bool up1 = softmax(NQB - 1, s1, p1, a1);
            if (j > 0 && __any(up1)) rescale(NQB - 1, a1);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) kf[kk] = kn[kk];
#pragma unroll
            for (int ts = 0; ts < 2; ++ts)
#pragma unroll
                for (int db = 0; db < 4; ++db) vprev[ts][db] = vf[ts][db];
        }
        pv(NQB - 1, vprev, p1);
    } else if (FULL) {
        // one query block: step j+1's scores and step j-1's PV under step j's softmax
        f32x16 s[2];
        bf16x8 pp[2][2], kf[KS], vprev[2][4];
        float a0;
        load_k(0, kf);
        qk(0, kf, s[0]);
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
            const int cur = j & 1, nxt = cur ^ 1;
            bf16x8 vf[2][4];
            if (j + 1 < NSTEP) {
                load_k(j + 1, kf);
                qk(0, kf, s[nxt]);
            }
            if (j == NSTEP - 2) {
                load_q_block<DK>(qf[0], p, b, h, q_next, q_next, lane);
                load_q_block<DK>(qf[1], p, b, h, q_next + 32, q_next, lane);
            }
            if (j > 0) pv(0, vprev, pp[nxt]);
            load_v(j, vf);
            const bool up = softmax(0, s[cur], pp[cur], a0);
            if (j > 0 && __any(up)) rescale(0, a0);
#pragma unroll
            for (int ts = 0; ts < 2; ++ts)
#pragma unroll
                for (int db = 0; db < 4; ++db) vprev[ts][db] = vf[ts][db];
        }
        pv(0, vprev, pp[(NSTEP - 1) & 1]);
    } else {
        for (int j = 0; j < nsub; ++j) {
            bf16x8 kf[KS], vf[2][4];
            load_k(j, kf);
            load_v(j, vf);
            const int vj = valid - 32 * j;
            int hfo = hf;  // opaque: keeps the mask constants out of the outer loop
            asm volatile("" : "+v"(hfo));
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                f32x16 s;
                bf16x8 pb[2];
                float a;
                qk(qb, kf, s);
                if (vj < 32) {
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (8 * (i >> 2) + 4 * hfo + (i & 3) >= vj) s[i] = -INFINITY;
                }
                const bool up = softmax(qb, s, pb, a);
                if (j > 0 && __any(up)) rescale(qb, a);
                pv(qb, vf, pb);
            }
        }
        load_q_block<DK>(qf[0], p, b, h, q_next, q_next, lane);
        load_q_block<DK>(qf[1], p, b, h, q_next + 32, q_next, lane);
    }

    // partial of this chunk: O / l (bf16) and m + log2(l).  Lane dword k of
    // a block holds o[db = k/8][2*(k%8) + {0, 1}] and is stored at
    // 1 KB * (k/4) + 16 B * lane + 4 B * (k%4): every store instruction
    // writes 1 KB contiguous.  Query columns past Q hold finite values
    // that the combine ignores.
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const float lt = halfwave_sum(l[qb]);
        const float inv = __builtin_amdgcn_rcpf(lt);  // the partial is rounded to bf16
        const int64_t blk = ((int64_t)bh * p.nch_total + chunk) * p.qblocks + (q0 >> 5) + qb;
        uint16_t* dst = p.part_o + blk * 4096 + lane * 8;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const int db = st >> 1, i0 = 8 * (st & 1);
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = pack_bf16x2(o[qb][db][i0 + 2 * e] * inv, o[qb][db][i0 + 2 * e + 1] * inv);
            NT_STORE(w, reinterpret_cast<u32x4*>(dst + 512 * st));
        }
        if (hf == 0)
            NT_STORE(m[qb] + log2f(lt),
                     p.part_lse + ((int64_t)bh * p.nch_total + chunk) * ((int64_t)p.qblocks * 32) +
                         q0 + 32 * qb + l32);
    }
}

template <int DK>
__global__ void __launch_bounds__(CK_THREADS, 1) chunk_kernel(ChunkParams p) {
    constexpr int KROW = KTile<DK>::ROW;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    ChunkSmem& sm = *reinterpret_cast<ChunkSmem*>(smem_raw);
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

    // block -> (bh, chunk) with bh fastest: with B*H a multiple of 8 all
    // chunks of one head run on one XCD (blocks go to the 8 XCDs
    // round-robin), sharing that head's decoder rows, centers and queries in
    // one L2.  History chunks come first; the cheaper current-chunk blocks
    // fill the tail.
    const int BH = p.B * p.H;
    const int bh = blockIdx.x % BH;
    const int chunk = blockIdx.x / BH;
    const int b = bh / p.H, h = bh % p.H;
    const bool hist = chunk < p.nch_hist;
    const int64_t tok0 = (int64_t)(hist ? chunk : chunk - p.nch_hist) * CK_T;
    const int valid = (int)min((int64_t)CK_T, (hist ? p.n_rows : p.Nc) - tok0);

    if (hist) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const ChunkCodec& cd = p.codec[cc];
            int id = 0;
            if (cd.centers && t < valid) {
                // ids outside the table are clamped so that a corrupt payload
                // cannot read out of bounds (valid payloads never hold them)
                const int64_t key = tok0 + t;
                id = read_id(cd.ids, cd.id_bytes, (int64_t)b * p.N + history_row(p, key));
                id = min(max(id, 0), cd.num_centers - 1);
            }
            sm.ids[cc][t] = id;
            const int width = cc == 0 ? DK : CK_D;
            if (t < width)
                sm.bias[cc][t] = cd.bias ? bf16_round(cd.bias[(int64_t)h * cd.bias_hs + t]) : 0.0f;
        }
        __syncthreads();
        // V first: its decoder slices are staged in the (not yet written)
        // V^T region and its centers in the wave's own K rows; then K, with
        // its slices staged in the K region once every wave has read its V
        // centers.
        uint16_t* vt_scratch = &sm.vt[0][0];
        uint16_t* k_scratch = &sm.k[0][0];
        if (p.codec[1].centers)
            decode_codec<1, true, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                              wave, lane);
        else
            decode_codec<1, false, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                               wave, lane);
        __syncthreads();
        if (p.codec[0].centers)
            decode_codec<0, true, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid, wave,
                                            lane);
        else
            decode_codec<0, false, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid,
                                             wave, lane);
    } else if (DK == CK_D) {
        load_current_chunk(sm, p, b, h, tok0, valid, t);
    }
    __syncthreads();

    const int nsub = (valid + 31) / 32;
    const int nqt = (int)cdiv(p.Q, CK_QT);
    constexpr int WAVES = CK_THREADS / 64;
    bf16x8 qf[2][8];
    if (wave < nqt) {
        load_q_block<DK>(qf[0], p, b, h, (int64_t)wave * CK_QT, (int64_t)wave * CK_QT, lane);
        load_q_block<DK>(qf[1], p, b, h, (int64_t)wave * CK_QT + 32, (int64_t)wave * CK_QT, lane);
    }
    for (int qt = wave; qt < nqt; qt += WAVES) {
        const int64_t q0 = (int64_t)qt * CK_QT;
        // the wave's next tile, or this one again (a harmless in-bounds reload)
        const int64_t q_next = qt + WAVES < nqt ? q0 + WAVES * CK_QT : q0;
        const bool one = q0 + 32 >= p.Q;
        if (valid == CK_T) {
            if (one) attend_qtile<DK, 1, true>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
            else attend_qtile<DK, 2, true>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
        } else {
            if (one) attend_qtile<DK, 1, false>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
            else attend_qtile<DK, 2, false>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
        }
    }
}

// Merge the chunk partials of every (b, h, q).  A 256-thread block owns one
// 32-query block; its four waves take every fourth chunk, each lane reading
// the lane-order payload the attention wave stored, and sum through LDS.
// out = sum_c 2^(lse_c - M) O_c / sum_c 2^(lse_c - M); no chunks give
// out = 0 and lse = -inf (CN/core.py:48-49).
constexpr int CB_WAVES = 4;
__global__ void __launch_bounds__(64 * CB_WAVES) chunk_combine_kernel(ChunkParams p) {
    __shared__ float red[CB_WAVES - 1][64][65];  // [wave-1][element][lane] (+1 pad)
    __shared__ float redl[CB_WAVES - 1][64];
    const int lane = threadIdx.x & 63, hf = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t bh = blockIdx.x / p.qblocks;
    const int qblk = (int)(blockIdx.x % p.qblocks);
    const int64_t qi = (int64_t)qblk * 32 + l32;
    const int NC = p.nch_total;
    const int64_t lse_stride = (int64_t)p.qblocks * 32;
    const float* lr = p.part_lse + bh * NC * lse_stride + qi;
    // eight independent maxima keep eight loads in flight
    float mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mx[e] = -INFINITY;
    int cc0 = 0;
    for (; cc0 + 8 <= NC; cc0 += 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) mx[e] = fmaxf(mx[e], lr[(cc0 + e) * lse_stride]);
    }
    for (; cc0 < NC; ++cc0) mx[0] = fmaxf(mx[0], lr[cc0 * lse_stride]);
    float M = mx[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) M = fmaxf(M, mx[e]);
    const float Mu = M == -INFINITY ? 0.0f : M;
    float L = 0.0f, acc[64];
#pragma unroll
    for (int e = 0; e < 64; ++e) acc[e] = 0.0f;
    const uint16_t* src = p.part_o + (bh * NC * p.qblocks + qblk) * 4096 + lane * 8;
    const int64_t cstride = (int64_t)p.qblocks * 4096;
#pragma unroll 2
    for (int cc = wave; cc < NC; cc += CB_WAVES) {
        const float wt = exp2f(lr[cc * lse_stride] - Mu);
        L += wt;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src + cc * cstride + 512 * st);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[8 * st + 2 * e] += wt * __uint_as_float(v[e] << 16);
                acc[8 * st + 2 * e + 1] += wt * __uint_as_float(v[e] & 0xffff0000u);
            }
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int e = 0; e < 64; ++e) red[wave - 1][e][lane] = acc[e];
        redl[wave - 1][lane] = L;
    }
    __syncthreads();
    if (wave > 0 || qi >= p.Q) return;
#pragma unroll
    for (int w = 0; w < CB_WAVES - 1; ++w) {
#pragma unroll
        for (int e = 0; e < 64; ++e) acc[e] += red[w][e][lane];
        L += redl[w][lane];
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const int b = (int)(bh / p.H), h = (int)(bh % p.H);
    uint16_t* orow = p.out + b * p.o_sb + qi * p.o_st + h * p.o_sh + 4 * hf;
    // acc[8*st + 2*e + {0,1}] = o[db = st/2][i = 8*(st&1) + 2*e + {0,1}] with
    // d = 32*db + 8*(i/4) + 4*hf + i%4: acc[4n .. 4n+3] are four consecutive
    // d of this lane's query
#pragma unroll
    for (int n = 0; n < 16; ++n) {
        const int st = n >> 1;
        const int db = st >> 1, i = 8 * (st & 1) + 4 * (n & 1);
        const int d = 32 * db + 8 * (i >> 2);
        const u32x2 pk = {pack_bf16x2(acc[4 * n] * inv, acc[4 * n + 1] * inv),
                          pack_bf16x2(acc[4 * n + 2] * inv, acc[4 * n + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = pk;
    }
    if (p.lse && hf == 0)
        p.lse[bh * p.Q + qi] = L > 0.0f ? (M + log2f(L)) * 0.69314718055994531f : -INFINITY;
}

// ------------------------------------------------------------------ host
ChunkCodec chunk_codec_from(const nkv_codec& c, int D, int HD) {
    ChunkCodec v{};
    v.packed = c.packed;
    v.scales = c.scales;
    v.ids = c.centers ? c.ids : nullptr;
    v.r = c.r;
    v.group = c.group;
    v.scale_dtype = c.scale_dtype;
    v.id_bytes = c.id_bytes;
    v.num_centers = c.num_centers;
    v.w = c.w_dec;
    v.w_hs = (int64_t)D * c.r;
    v.centers = c.centers;
    v.c_bs = c.centers_batch_stride;
    v.c_rs = HD;
    v.c_hs = D;
    v.bias = c.mean;
    v.bias_hs = D;
    return v;
}

namespace {

int64_t chunk_count(int64_t keys) { return cdiv(keys, CK_T); }

int check_chunk_codec(const ChunkCodec& c) {
    NKV_REQUIRE(c.packed && c.scales && c.w, NKV_ERR_INVALID,
                "history codec needs packed codes, scales and decode rows");
    NKV_REQUIRE(c.r > 0 && c.r % 64 == 0 && c.r <= 4096, NKV_ERR_UNSUPPORTED,
                "key-chunk attend needs codec ranks that are multiples of 64");
    NKV_REQUIRE(c.group > 0 && c.group % 32 == 0 && c.r % c.group == 0, NKV_ERR_UNSUPPORTED,
                "key-chunk attend needs scale groups that are multiples of 32 dividing r");
    NKV_REQUIRE(c.scale_dtype == NKV_DTYPE_BF16 || c.scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    if (c.centers) {
        NKV_REQUIRE(c.ids && (c.id_bytes == 1 || c.id_bytes == 2 || c.id_bytes == 4),
                    NKV_ERR_INVALID, "centers need ids of 1, 2 or 4 bytes");
        NKV_REQUIRE(c.num_centers > 0, NKV_ERR_INVALID, "num_centers must be > 0");
    }
    return NKV_OK;
}

template <int DK>
void launch_dk(const ChunkParams& p, int64_t blocks, hipStream_t s, int* rc) {
    const size_t smem = sizeof(ChunkSmem);
    hipError_t e = hipFuncSetAttribute((const void*)chunk_kernel<DK>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
        set_error(std::string("chunk_launch: hipFuncSetAttribute failed: ") + hipGetErrorString(e));
        *rc = NKV_ERR_HIP;
        return;
    }
    chunk_kernel<DK><<<dim3((unsigned)blocks), CK_THREADS, smem, s>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string("chunk_launch: launch failed: ") + hipGetErrorString(e));
        *rc = NKV_ERR_HIP;
    }
}

}  // namespace

size_t chunk_launch_workspace(const ChunkLaunchDesc& d) {
    const int64_t nc = chunk_count(d.n_rows) + chunk_count(d.Nc);
    const size_t blocks = (size_t)d.B * d.H * nc * cdiv(d.Q, 32);
    return blocks * 32 * CK_D * sizeof(uint16_t) + blocks * 32 * sizeof(float);
}

int chunk_launch(hipStream_t s, const ChunkLaunchDesc& d, void* workspace, size_t workspace_bytes) {
    NKV_REQUIRE(d.dk == 32 || d.dk == 64 || d.dk == 128, NKV_ERR_UNSUPPORTED,
                "key-chunk attend supports K/Q widths 32, 64 and 128");
    NKV_REQUIRE(d.B >= 1 && d.H >= 1 && d.Q >= 0 && d.n_rows >= 0 && d.Nc >= 0, NKV_ERR_INVALID,
                "bad launch shape");
    NKV_REQUIRE(d.Nc == 0 || (d.dk == CK_D && d.k_cur && d.v_cur), NKV_ERR_INVALID,
                "current keys need k_cur/v_cur and a 128-wide launch");
    if (d.n_rows > 0) {
        int rc = check_chunk_codec(d.key);
        if (rc) return rc;
        rc = check_chunk_codec(d.value);
        if (rc) return rc;
    }
    if (d.Q == 0) return NKV_OK;
    NKV_REQUIRE(d.q && d.out, NKV_ERR_INVALID, "q and out required");
    const size_t need = chunk_launch_workspace(d);
    NKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), NKV_ERR_WORKSPACE,
                "workspace missing or smaller than the size query returned");
    ChunkParams p;
    p.B = d.B;
    p.H = d.H;
    p.nch_hist = (int)chunk_count(d.n_rows);
    p.nch_total = p.nch_hist + (int)chunk_count(d.Nc);
    p.qblocks = (int)cdiv(d.Q, 32);
    p.Q = d.Q;
    p.N = d.N;
    p.n_rows = d.n_rows;
    p.rows = d.rows;
    p.Nc = d.Nc;
    p.scale_log2 = d.softmax_scale * 1.4426950408889634f;
    p.q = d.q;
    p.q_sb = d.q_sb;
    p.q_st = d.q_st;
    p.q_sh = d.q_sh;
    p.k_cur = d.k_cur;
    p.k_sb = d.k_sb;
    p.k_st = d.k_st;
    p.k_sh = d.k_sh;
    p.v_cur = d.v_cur;
    p.v_sb = d.v_sb;
    p.v_st = d.v_st;
    p.v_sh = d.v_sh;
    p.codec[0] = d.key;
    p.codec[1] = d.value;
    const size_t qrows = (size_t)d.B * d.H * p.nch_total * p.qblocks * 32;
    p.part_o = reinterpret_cast<uint16_t*>(workspace);
    p.part_lse = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) +
                                          qrows * CK_D * sizeof(uint16_t));
    p.out = d.out;
    p.o_sb = d.o_sb;
    p.o_st = d.o_st;
    p.o_sh = d.o_sh;
    p.lse = d.lse;

    const int64_t blocks = (int64_t)d.B * d.H * p.nch_total;
    if (d.ev_begin) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d.ev_begin, s));
    if (blocks > 0) {
        int rc = NKV_OK;
        if (d.dk == 128) launch_dk<128>(p, blocks, s, &rc);
        else if (d.dk == 64) launch_dk<64>(p, blocks, s, &rc);
        else launch_dk<32>(p, blocks, s, &rc);
        if (rc) return rc;
    }
    if (d.ev_end) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d.ev_end, s));
    const int64_t qblocks_total = (int64_t)d.B * d.H * p.qblocks;
    if (qblocks_total > 0) {
        chunk_combine_kernel<<<dim3((unsigned)qblocks_total), 64 * CB_WAVES, 0, s>>>(p);
        NKV_LAUNCH_CHECK();
    }
    return NKV_OK;
}

// nkv_attend's key-chunk path: every head, all history rows, decoder tables.
namespace {
ChunkLaunchDesc desc_from(const nkv_attend_args* a) {
    ChunkLaunchDesc d{};
    d.B = a->B;
    d.H = a->H;
    d.dk = a->D;
    d.Q = a->Q;
    d.N = a->N;
    d.n_rows = a->N;
    d.rows = nullptr;
    d.Nc = a->Nc;
    d.softmax_scale = a->softmax_scale;
    d.q = a->q;
    d.q_sb = a->q_sb;
    d.q_st = a->q_st;
    d.q_sh = a->q_sh;
    d.k_cur = a->k_cur;
    d.k_sb = a->k_sb;
    d.k_st = a->k_st;
    d.k_sh = a->k_sh;
    d.v_cur = a->v_cur;
    d.v_sb = a->v_sb;
    d.v_st = a->v_st;
    d.v_sh = a->v_sh;
    const int HD = a->H * a->D;
    d.key = chunk_codec_from(a->key, a->D, HD);
    d.value = chunk_codec_from(a->value, a->D, HD);
    d.out = a->out;
    d.o_sb = a->o_sb;
    d.o_st = a->o_st;
    d.o_sh = a->o_sh;
    d.lse = a->lse;
    d.ev_begin = a->ev_kernel_begin;
    d.ev_end = a->ev_kernel_end;
    return d;
}
}  // namespace

size_t chunk_workspace_bytes(const nkv_attend_args* a) { return chunk_launch_workspace(desc_from(a)); }

int chunk_check(const nkv_attend_args* a) {
    NKV_REQUIRE(a->D == CK_D, NKV_ERR_UNSUPPORTED, "key-chunk attend supports D == 128");
    if (a->N > 0) {
        for (const nkv_codec* c : {&a->key, &a->value}) {
            NKV_REQUIRE(c->r > 0 && c->r % 64 == 0 && c->r <= 4096, NKV_ERR_UNSUPPORTED,
                        "key-chunk attend needs codec ranks that are multiples of 64");
            NKV_REQUIRE(c->group % 32 == 0, NKV_ERR_UNSUPPORTED,
                        "key-chunk attend needs scale groups that are multiples of 32");
        }
    }
    return NKV_OK;
}

int chunk_attend_launch(hipStream_t s, const nkv_attend_args* a, void* workspace,
                        size_t workspace_bytes) {
    int rc = chunk_check(a);
    if (rc) return rc;
    return chunk_launch(s, desc_from(a), workspace, workspace_bytes);
}

}  // namespace nkv
