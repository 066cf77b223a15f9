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

#include <type_traits>

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
    float* part_ml;     // [B*H, nch_total, qblocks * 32, 2]: running max (log2 units), row sum
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
//
// Decoder slices W[row d of the launch head][64*s, +64) (WIDTH rows of 128
// bytes) stream into a ring of DS_NBUF LDS buffers by direct-to-LDS loads
// (global_load_lds_dwordx4: no register staging), DS_AHEAD slices ahead of
// the MFMAs.  The block's four waves each copy WIDTH/32 KB of a slice, so
// every decoder element is fetched from L2 once per block.  Rows are stored
// unpadded with their 16-byte chunks XOR-swizzled by (row & 7): chunk c of
// row r sits at chunk c ^ (r & 7), so the MFMA operand reads of eight
// consecutive rows hit eight distinct chunks (conflict-free), while every
// load instruction still fills one contiguous 1 KB of LDS.
//
// A stage (slice s) = its decoder rows plus this wave's codes and scales of
// slice s, which go to a register ring of DS_AHEAD entries.  Loads complete
// in issue order, so waiting for stage s is one vmcnt bound: the stages
// issued after it may stay in flight.
constexpr int DS_NBUF = 4;
constexpr int DS_AHEAD = 3;
// The rings fit in the regions that hold no live data while they are used:
// V's decode stages in the V^T region, K's in the K region.
static_assert(DS_NBUF * CK_D * 64 <= CK_D * CK_VROW && DS_NBUF * CK_D * 64 <= CK_T * CK_KROW,
              "decoder staging must fit in the V^T and K regions");
static_assert(CK_T * CK_D <= CK_T * CK_KROW, "V centers are staged in the K region");

#define NKV_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits [3:0] and [15:14]; the
// other counters at their maxima, i.e. not waited on)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The 128 center values of launch head h for the wave's 64 keys (V), copied
// into LDS rows [key][128] (unpadded, key 64*wave + ... of the chunk) by
// 16 direct-to-LDS loads, each filling 4 rows (1 KB).
__device__ __forceinline__ void dma_v_centers(uint16_t* vcen, const ChunkSmem& sm,
                                              const ChunkCodec& c, int b, int h, int wave,
                                              int lane) {
    const uint16_t* cent = c.centers + (int64_t)b * c.c_bs + (int64_t)h * c.c_hs + 8 * (lane & 15);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int t = 64 * wave + 4 * e + (lane >> 4);
        __builtin_amdgcn_global_load_lds(cent + (int64_t)sm.ids[1][t] * c.c_rs,
                                         NKV_LDS(vcen + (64 * wave + 4 * e) * CK_D), 16, 0, 0);
    }
}

// The DK center values of launch head h for the wave's 64 keys (K), as
// coalesced 16-byte row pieces: entry e of lane L is piece q = 64*e + L of
// the wave's rows, i.e. key 64*wave + q / (DK/8) of the chunk, columns
// 8 * (q % (DK/8)).
template <int DK>
__device__ __forceinline__ void load_k_center_rows(u32x4 (&v)[DK / 8], const ChunkSmem& sm,
                                                   const ChunkCodec& c, int b, int h, int wave,
                                                   int lane) {
    constexpr int PR = DK / 8;  // 16-byte pieces per row
    const uint16_t* cent = c.centers + (int64_t)b * c.c_bs + (int64_t)h * c.c_hs;
#pragma unroll
    for (int e = 0; e < DK / 8; ++e) {
        const int q = 64 * e + lane;  // piece index within the wave's 64 rows
        const int t = 64 * wave + q / PR;
        v[e] = *reinterpret_cast<const u32x4*>(cent + (int64_t)sm.ids[0][t] * c.c_rs +
                                               8 * (q % PR));
    }
}

// Decode this wave's 64 keys of codec CODEC to WIDTH columns (V: 128, into
// V^T; K: the launch's DK, into the K tile with row pitch KROW).  wst: the
// LDS ring (DS_NBUF * WIDTH * 64 bf16) that holds no live data during the
// call.  HAS_C: the codec has centers (a template argument so that the
// epilogue is straight-line code); V's are copied into the K region
// (unpadded rows) after `pre`, K's are loaded into registers before the
// slices.  pre() runs once the first stages are in flight (V: it publishes
// the chunk's ids and biases, ending with a block barrier).  Ends with a
// block barrier.
template <int CODEC, bool HAS_C, int WIDTH, int KROW, typename Pre>
__device__ __forceinline__ void decode_codec(ChunkSmem& sm, uint16_t* wst, const ChunkCodec& c,
                                             const ChunkParams& p, int b, int h, int64_t tok0,
                                             int valid, int wave, int lane, Pre&& pre) {
    constexpr int NDT = WIDTH / 32;
    constexpr int LPW = WIDTH / 32;           // 1 KB slice loads per wave
    constexpr int STAGE = LPW + 4;            // vm instructions per stage
    constexpr int SLICE = WIDTH * 64;         // bf16 per ring buffer
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
    // slice loads: this wave fills 1 KB pieces 4*wave*.. of each slice; lane
    // L brings logical chunk (L%8) ^ (L/8) of row 8*piece + L/8
    const int piece_row = lane >> 3, piece_chunk = (lane & 7) ^ (lane >> 3);
    const uint16_t* wsrc = c.w + (int64_t)h * c.w_hs + (int64_t)piece_row * R + 8 * piece_chunk;
    auto issue_slice = [&](int s) {
        uint16_t* dst = wst + (s % DS_NBUF) * SLICE;
#pragma unroll
        for (int e = 0; e < LPW; ++e) {
            const int piece = LPW * wave + e;  // rows 8*piece .. +8
            __builtin_amdgcn_global_load_lds(wsrc + (int64_t)8 * piece * R + 64 * s,
                                             NKV_LDS(dst + piece * 512), 16, 0, 0);
        }
    };
    // codes and raw scale bits (converted at use: converting here would make
    // the issue wait for the load)
    auto issue_codes = [&](int s, u32x4 (&pk)[2], uint16_t (&sb)[2]) {
        const int gi = (64 * s + 32 * hf) / G;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            pk[tt] = *reinterpret_cast<const u32x4*>(prow[tt] + 32 * s);
            sb[tt] = srow[tt][gi];
        }
    };

    f32x16 acc[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[dt][tt] = f32x16{};

    // K: center rows, issued before stage 0 (so complete before it)
    uint16_t* vcen = &sm.k[0][0];
    u32x4 kcen[WIDTH / 8];
    if (CODEC == 0 && HAS_C) load_k_center_rows<WIDTH>(kcen, sm, c, b, h, wave, lane);

    u32x4 pk[DS_AHEAD][2];
    uint16_t sc[DS_AHEAD][2];
    // (sched_barrier: the stages must leave in this order, since the vmcnt
    // bounds below count whole stages)
#pragma unroll
    for (int i = 0; i < DS_AHEAD; ++i)
        if (i < KQ) {
            issue_slice(i);
            issue_codes(i, pk[i], sc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    pre();
    // V: center rows into the K region, issued after stages 0 .. DS_AHEAD-1
    // and before stage DS_AHEAD: NVC more instructions may be in flight while
    // waiting for the first DS_AHEAD stages
    constexpr int NVC = CODEC == 1 && HAS_C ? 16 : 0;
    if (CODEC == 1 && HAS_C) dma_v_centers(vcen, sm, c, b, h, wave, lane);
    __builtin_amdgcn_sched_barrier(0);

    // per-lane swizzled chunk offsets of the operand reads: row 32*dt + l32,
    // logical chunk 4*hf + j
    int wofs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wofs[j] = l32 * 64 + 8 * ((4 * hf + j) ^ (l32 & 7));

    // operand of the current sub-step (carried across slices), and its scales
    u32x4 zc[2];
    float scl[2], ns7[2];
    if (KQ > 0) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            scl[tt] = f16 ? f16_bits_to_f32(sc[0][tt]) : bf16_bits_to_f32(sc[0][tt]);
            ns7[tt] = -7.0f * scl[tt];
            Unpack8 u;
            u.split(pk[0][tt][0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) zc[tt][e] = u.pair(e, scl[tt], ns7[tt]);
        }
    }
    for (int s0 = 0; s0 < KQ; s0 += DS_AHEAD) {
#pragma unroll
        for (int i = 0; i < DS_AHEAD; ++i) {
            const int s = s0 + i;
            if (s >= KQ) break;
            // stage s landed (for this wave) once at most the later issued
            // stages are in flight; the barrier makes every wave's part visible
            // and retires the reads of the buffer the next slice goes to
            static_assert(DS_AHEAD == 3, "the wait bounds below assume three stages ahead");
            const int later = min(KQ - 1 - s, DS_AHEAD - 1);
            if (s < DS_AHEAD) {
                if (later >= 2) wait_vmcnt<2 * STAGE + NVC>();
                else if (later == 1) wait_vmcnt<STAGE + NVC>();
                else wait_vmcnt<NVC>();
            } else {
                if (later >= 2) wait_vmcnt<2 * STAGE>();
                else if (later == 1) wait_vmcnt<STAGE>();
                else wait_vmcnt<0>();
            }
            __builtin_amdgcn_s_barrier();
            if (s + DS_AHEAD < KQ) issue_slice(s + DS_AHEAD);
            __builtin_amdgcn_sched_barrier(0);
            const uint16_t* wb = wst + (s % DS_NBUF) * SLICE;
            // Software pipeline in explicit slots: each MFMA of sub-step j is
            // followed by one eighth of the next sub-step's unpack (for the
            // last sub-step: the next slice's first, whose codes are already
            // in the ring) and, every other slot, one of the next sub-step's
            // decoder-operand reads (not across slices: those need the
            // barrier); sched_barrier keeps the slots in order so that the
            // unpack runs under the MFMAs.
            // (after the last slice the ring entry holds stale codes: the
            // unpack is then wasted work, kept branch-free)
            const int inx = (i + 1) % DS_AHEAD;
            float scn[2], nsn[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                scn[tt] = f16 ? f16_bits_to_f32(sc[inx][tt]) : bf16_bits_to_f32(sc[inx][tt]);
                nsn[tt] = -7.0f * scn[tt];
            }
            u32x4 zn[2];
            bf16x8 wc[NDT], wn[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) wc[dt] = lds_b128(wb + 32 * dt * 64 + wofs[0]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                Unpack8 u[2];
                constexpr int SLOTS = 2 * NDT;  // MFMAs per sub-step
#pragma unroll
                for (int m = 0; m < SLOTS; ++m) {
                    const int dt = m >> 1, tt = m & 1;
                    acc[dt][tt] = CODEC == 0 ? mfma32(wc[dt], as_bf16x8(zc[tt]), acc[dt][tt])
                                             : mfma32(as_bf16x8(zc[tt]), wc[dt], acc[dt][tt]);
                    // unpack pieces: 8 dwords (2 tt x 4) over the SLOTS slots
#pragma unroll
                    for (int q = (8 * m) / SLOTS; q < (8 * (m + 1)) / SLOTS; ++q) {
                        const int qt = q >> 2, qe = q & 3;
                        if (j + 1 < 4) {
                            if (qe == 0) u[qt].split(pk[i][qt][j + 1]);
                            zn[qt][qe] = u[qt].pair(qe, scl[qt], ns7[qt]);
                        } else {
                            if (qe == 0) u[qt].split(pk[inx][qt][0]);
                            zn[qt][qe] = u[qt].pair(qe, scn[qt], nsn[qt]);
                            // computed here, under this slice's MFMAs (the
                            // compiler would otherwise sink it past the barrier)
                            asm volatile("" : "+v"(zn[qt][qe]));
                        }
                    }
                    if (j + 1 < 4 && (m & 1) == 0)
                        wn[dt] = lds_b128(wb + 32 * dt * 64 + wofs[j + 1]);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) zc[tt] = zn[tt];
                if (j + 1 < 4) {
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) wc[dt] = wn[dt];
                }
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                scl[tt] = scn[tt];
                ns7[tt] = nsn[tt];
            }
            // this ring entry is consumed: refill it with stage s + DS_AHEAD
            __builtin_amdgcn_sched_barrier(0);
            if (s + DS_AHEAD < KQ) issue_codes(s + DS_AHEAD, pk[i], sc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // every wave's slice reads are done before the epilogue writes over the ring
    __syncthreads();

    // Epilogue.  sm.bias holds bf16(mean) or zeros, so the bias add is
    // unconditional.
    if (CODEC == 0) {
        // acc[dt][tt] element i: d = 32*dt + 8*(i/4) + 4*hf + i%4, key
        // 64*wave + 32*tt + l32.  Pass 1 stores bf16(acc + bias) ...
        uint16_t* ktile = &sm.k[0][0];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 64 * wave + 32 * tt + l32;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * dt + 8 * g + 4 * hf;
                    float a[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) a[e] = acc[dt][tt][4 * g + e] + sm.bias[0][d + e];
                    const u32x2 r = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
                    *reinterpret_cast<u32x2*>(ktile + t * KROW + d) = r;
                }
        }
        if (HAS_C) {
            // ... pass 2 adds the center rows piece by piece (the wave's own
            // rows: its LDS operations stay in order, no barrier needed)
            constexpr int PR = WIDTH / 8;
#pragma unroll
            for (int e = 0; e < WIDTH / 8; ++e) {
                const int q = 64 * e + lane;
                u32x4* slot = reinterpret_cast<u32x4*>(ktile + (64 * wave + q / PR) * KROW +
                                                       8 * (q % PR));
                const u32x4 kv = *slot;
                u32x4 r;
#pragma unroll
                for (int h2 = 0; h2 < 4; ++h2)
                    r[h2] = pack_bf16x2(
                        __uint_as_float(kv[h2] << 16) + __uint_as_float(kcen[e][h2] << 16),
                        __uint_as_float(kv[h2] & 0xffff0000u) +
                            __uint_as_float(kcen[e][h2] & 0xffff0000u));
                *slot = r;
            }
        }
    } else {
        // acc[dt][tt] element i: key 64*wave + 32*tt + 8*(i/4) + 4*hf + i%4, d = 32*dt + l32;
        // the center rows of the wave's keys are in vcen
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
                        v[e] = HAS_C ? a + bf16_bits_to_f32(vcen[(t0 + e) * CK_D + d]) : a;
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
template <int DK, int NF>
__device__ __forceinline__ void load_q_block(bf16x8 (&qf)[NF], const ChunkParams& p, int b, int h,
                                             int64_t q_blk, int64_t q_safe, int lane) {
    using W = DWalk<DK>;
    static_assert(NF >= W::KSTEPS, "fragment array too small");
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
// The partial of one 32-query block for this chunk: its O (unnormalised,
// bf16) and per query the running max m (log2 units) and row sum l, so that
// the combine forms sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.  Lane
// dword k of the block holds o[db = k/8][2*(k%8) + {0, 1}] and is stored at
// 1 KB * (k/4) + 16 B * lane + 4 B * (k%4): every store instruction writes
// 1 KB contiguous.  Query columns past Q hold finite values that the combine
// ignores; both half-waves store the same (m, l) of their query.
__device__ __forceinline__ void store_partial_piece(const ChunkParams& p, int64_t blk,
                                                    const f32x16 (&o)[4], int st, int lane) {
    uint16_t* dst = p.part_o + blk * 4096 + lane * 8;
    const int db = st >> 1, i0 = 8 * (st & 1);
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(o[db][i0 + 2 * e], o[db][i0 + 2 * e + 1]);
    NT_STORE(w, reinterpret_cast<u32x4*>(dst + 512 * st));
}

__device__ __forceinline__ void store_partial_ml(const ChunkParams& p, int64_t bh, int chunk,
                                                 int64_t qcol, float m, float lt) {
    const int64_t idx = (bh * p.nch_total + chunk) * ((int64_t)p.qblocks * 32) + qcol;
    NT_STORE((u32x2{__float_as_uint(m), __float_as_uint(lt)}),
             reinterpret_cast<u32x2*>(p.part_ml + 2 * idx));
}

__device__ __forceinline__ void store_partial(const ChunkParams& p, int64_t bh, int chunk,
                                              int64_t qblk0, const f32x16 (&o)[4], float m,
                                              float lt, int lane) {
    const int64_t blk = ((int64_t)bh * p.nch_total + chunk) * p.qblocks + (qblk0 >> 5);
#pragma unroll
    for (int st = 0; st < 8; ++st) store_partial_piece(p, blk, o, st, lane);
    store_partial_ml(p, bh, chunk, qblk0 + (lane & 31), m, lt);
}

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
        // Two query blocks staggered by half a step.  Every phase issues up
        // to 16 MFMAs that do not depend on its softmax (one block's scores
        // of the next step, the other block's PV) and spreads that softmax
        // between them, one slice per MFMA, with the next operands' LDS
        // loads riding along; sched_barrier fences keep this order, so one
        // wave keeps the matrix core busy while it runs the softmax.
        //   X(j): S1 = QK(K_j), O1 += PV(V_{j-1}, P1) | softmax(S0) | load K_{j+1}
        //   Y(j): S0 = QK(K_{j+1}), O0 += PV(V_j, P0) | softmax(S1) | load V_{j+1}
        f32x16 s0, s1;
        bf16x8 p0[2], p1[2];
        bf16x8 kb[2][KS], vb[2][2][4];
        float a0 = 1.0f, a1 = 1.0f;
        load_k(0, kb[0]);
        load_v(0, vb[0]);
        qk(0, kb[0], s0);
        // one phase; NQK / NPV = MFMAs of the score / PV product (0 = none)
        auto phase = [&](auto nqk_c, auto npv_c, const bf16x8 (&kq)[KS], int qa, f32x16& s_out,
                         const bf16x8 (&vv)[2][4], int qv, const bf16x8 (&pin)[2], int qs,
                         f32x16& s_in, bf16x8 (&pout)[2], float& alpha, auto&& ld) -> bool {
            constexpr int NQK = decltype(nqk_c)::value, NPV = decltype(npv_c)::value;
            constexpr int BOTH = NQK < NPV ? NQK : NPV;
            const float mq = m[qs];
            float tm = 0.0f, mn = 0.0f, lsum = 0.0f;
            bool up = false;
            uint32_t pw[8];
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                // MFMA t: score and PV products alternate, then the longer one's tail
                int kind = -1, idx = 0;  // 0: score step idx, 1: PV step idx
                if (t < 2 * BOTH) {
                    kind = t & 1;
                    idx = t >> 1;
                } else if (t - BOTH < NQK && NQK > BOTH) {
                    kind = 0;
                    idx = t - BOTH;
                } else if (t - BOTH < NPV && NPV > BOTH) {
                    kind = 1;
                    idx = t - BOTH;
                }
                if (kind == 0) {
                    s_out = mfma32(kq[idx], qf[qa][idx], idx == 0 ? f32x16{} : s_out);
                } else if (kind == 1) {
                    const int ts = idx >> 2, db = idx & 3;
                    o[qv][db] = mfma32(vv[ts][db], pin[ts], o[qv][db]);
                }
                // softmax slice t (the max is taken on raw scores: c > 0 preserves order)
                if (t < 4) {
                    const float a = fmaxf(s_in[4 * t], s_in[4 * t + 1]);
                    const float b2 = fmaxf(s_in[4 * t + 2], s_in[4 * t + 3]);
                    tm = t == 0 ? fmaxf(a, b2) : fmaxf(tm, fmaxf(a, b2));
                } else if (t == 4) {
                    tm = halfwave_max(tm) * c;
                    up = tm > mq + CK_TAU;
                    mn = up ? tm : mq;
                    alpha = up ? __builtin_amdgcn_exp2f(mq - mn) : 1.0f;
                    m[qs] = mn;
                } else if (t < 13) {
                    // v_exp_f32 of arguments <= 8; results below 2^-126 flush to 0
                    const int k = t - 5;
                    const float e0 = __builtin_amdgcn_exp2f(fmaf(s_in[2 * k], c, -mn));
                    const float e1 = __builtin_amdgcn_exp2f(fmaf(s_in[2 * k + 1], c, -mn));
                    pw[k] = pack_bf16x2(e0, e1);
                } else if (t < 15) {
                    // row sum of the bf16 weights the PV product uses
#pragma unroll
                    for (int k = 4 * (t - 13); k < 4 * (t - 13) + 4; ++k)
                        lsum = __builtin_amdgcn_fdot2_f32_bf16(
                            __builtin_bit_cast(bf16x2, pw[k]),
                            __builtin_bit_cast(bf16x2, 0x3F803F80u), lsum, false);
                } else {
                    l[qs] = l[qs] * alpha + lsum;
                    asm volatile("" : "+v"(l[qs]));
                    pout[0] = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
                    pout[1] = as_bf16x8(u32x4{pw[4], pw[5], pw[6], pw[7]});
                }
                ld(t);
                __builtin_amdgcn_sched_barrier(0);
            }
            return up;
        };
        using I0 = std::integral_constant<int, 0>;
        using IK = std::integral_constant<int, KS>;
        using I8 = std::integral_constant<int, 8>;
        auto no_load = [](int) {};
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
            const int cj = j & 1, nj = cj ^ 1;
            auto ld_k = [&](int t) {
                if (j + 1 < NSTEP && t < KS) kb[nj][t] = lds_b128(kbase + 32 * (j + 1) * KROW + W::block(t));
            };
            auto ld_v = [&](int t) {
                if (j + 1 < NSTEP && t < 8)
                    vb[nj][t >> 2][t & 3] =
                        lds_2x64(vbase + 32 * (t & 3) * CK_VROW + 32 * (j + 1) + 16 * (t >> 2));
            };
            bool up0;
            if (j == 0)
                up0 = phase(IK{}, I0{}, kb[cj], 1, s1, vb[nj], 1, p1, 0, s0, p0, a0, ld_k);
            else
                up0 = phase(IK{}, I8{}, kb[cj], 1, s1, vb[nj], 1, p1, 0, s0, p0, a0, ld_k);
            if (j == NSTEP - 1) load_q_block<DK>(qf[1], p, b, h, q_next + 32, q_next, lane);
            if (j > 0 && __any(up0)) rescale(0, a0);
            bool up1;
            if (j + 1 < NSTEP)
                up1 = phase(IK{}, I8{}, kb[nj], 0, s0, vb[cj], 0, p0, 1, s1, p1, a1, ld_v);
            else
                up1 = phase(I0{}, I8{}, kb[nj], 0, s0, vb[cj], 0, p0, 1, s1, p1, a1, no_load);
            if (j == NSTEP - 2) load_q_block<DK>(qf[0], p, b, h, q_next, q_next, lane);
            if (j > 0 && __any(up1)) rescale(1, a1);
        }
        pv(1, vb[(NSTEP - 1) & 1], p1);
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

    // partial of this chunk
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb)
        store_partial(p, bh, chunk, q0 + 32 * qb, o[qb], m[qb], halfwave_sum(l[qb]), lane);
}

// All of a wave's two-block query tiles of a full chunk as one pipeline.
// Within a tile the 16 phases are those of attend_qtile's two-block path
// (X(j): S1 = QK(K_j), O1 += PV(V_{j-1}), softmax(S0); Y(j): S0 =
// QK(K_{j+1}), O0 += PV(V_j), softmax(S1)).  Across tiles there is no
// seam: Y(7) computes the next tile's first scores (K_0 with the next
// queries), X(0) adds the previous tile's last PV, and the previous tile's
// partials are stored from X(0) (block 0) and Y(0) (block 1), spread over
// their MFMA slots.  Each phase issues up to 16 MFMAs that do not depend on
// its softmax, with the softmax, the LDS loads of the next operands and any
// store work in between, one slice per MFMA (sched_barrier keeps the order),
// so that one wave keeps the matrix core busy.
//
// Tile i covers queries (wave + 4 i) * 64 + [0, 64); every tile must have
// both blocks (q0 + 32 < Q).  The first tile's "previous partials" are
// stored into its own slots, which its real partials overwrite later (same
// wave, same addresses, program order).
template <int DK>
__device__ __forceinline__ void attend_stream(const ChunkSmem& sm, const ChunkParams& p, int b,
                                              int h, int bh, int chunk, int wave, int lane_in,
                                              int ntiles) {
    int lane = lane_in;
    asm volatile("" : "+v"(lane));
    const int hf = lane >> 5, l32 = lane & 31;
    const float c = p.scale_log2;
    using W = DWalk<DK>;
    constexpr int KROW = KTile<DK>::ROW;
    constexpr int KS = W::KSTEPS;
    constexpr int NSTEP = CK_T / 32;
    uint32_t koff = l32 * KROW + W::HALF * hf, voff = l32 * CK_VROW + 4 * hf;
    asm volatile("" : "+v"(koff));
    asm volatile("" : "+v"(voff));
    const uint16_t* kbase = &sm.k[0][0] + koff;
    const uint16_t* vbase = &sm.vt[0][0] + voff;
    const int64_t part_blk = ((int64_t)bh * p.nch_total + chunk) * p.qblocks;
    auto tile_q0 = [&](int i) { return (int64_t)(wave + 4 * i) * CK_QT; };

    f32x16 o[2][4];
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int db = 0; db < 4; ++db) o[qb][db] = f32x16{};
    f32x16 s0, s1;
    bf16x8 p0[2], p1[2];
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) p0[ts] = p1[ts] = bf16x8{};
    bf16x8 kb[2][KS], vb[2][2][4];
    bf16x8 qf[2][KS], qn[2][KS];  // this tile's and the next tile's query fragments

    auto lds_k = [&](int j, int kk) { return lds_b128(kbase + 32 * j * KROW + W::block(kk)); };
    auto lds_v = [&](int j, int t) {
        return lds_2x64(vbase + 32 * (t & 3) * CK_VROW + 32 * j + 16 * (t >> 2));
    };
    {
        const int64_t q0 = tile_q0(0);
        load_q_block<DK>(qf[0], p, b, h, q0, q0, lane);
        load_q_block<DK>(qf[1], p, b, h, q0 + 32, q0, lane);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kb[0][kk] = lds_k(0, kk);
#pragma unroll
        for (int t = 0; t < 8; ++t) vb[0][t >> 2][t & 3] = lds_v(0, t);
        s0 = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) s0 = mfma32(kb[0][kk], qf[0][kk], s0);
    }

    // One phase.  NQK / NPV: MFMAs of the score / PV product (0 = none); ZPV:
    // the PV product starts a new O (zero accumulator); FRESH: the softmax
    // starts a new row state.  ld(t) / ext(t) add slot t's loads / extra work.
    auto phase = [&](auto nqk_c, auto npv_c, auto zpv_c, auto fresh_c,
                     const bf16x8 (&kq)[KS], const bf16x8 (&qsrc)[KS], f32x16& s_out,
                     const bf16x8 (&vv)[2][4], int qv, const bf16x8 (&pin)[2], int qs,
                     f32x16& s_in, bf16x8 (&pout)[2], float& alpha, auto&& ld,
                     auto&& ext) -> bool {
        constexpr int NQK = decltype(nqk_c)::value, NPV = decltype(npv_c)::value;
        constexpr bool ZPV = decltype(zpv_c)::value, FRESH = decltype(fresh_c)::value;
        constexpr int BOTH = NQK < NPV ? NQK : NPV;
        const float mq = FRESH ? -INFINITY : m[qs];
        float tm = 0.0f, mn = 0.0f, lsum = 0.0f;
        bool up = false;
        uint32_t pw[8];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            int kind = -1, idx = 0;  // 0: score step idx, 1: PV step idx
            if (t < 2 * BOTH) {
                kind = t & 1;
                idx = t >> 1;
            } else if (t - BOTH < NQK && NQK > BOTH) {
                kind = 0;
                idx = t - BOTH;
            } else if (t - BOTH < NPV && NPV > BOTH) {
                kind = 1;
                idx = t - BOTH;
            }
            if (kind == 0) {
                s_out = mfma32(kq[idx], qsrc[idx], idx == 0 ? f32x16{} : s_out);
            } else if (kind == 1) {
                const int ts = idx >> 2, db = idx & 3;
                o[qv][db] = mfma32(vv[ts][db], pin[ts], ZPV && ts == 0 ? f32x16{} : o[qv][db]);
            }
            // softmax slice t (the max is taken on raw scores: c > 0 preserves order)
            if (t < 4) {
                const float a = fmaxf(s_in[4 * t], s_in[4 * t + 1]);
                const float b2 = fmaxf(s_in[4 * t + 2], s_in[4 * t + 3]);
                tm = t == 0 ? fmaxf(a, b2) : fmaxf(tm, fmaxf(a, b2));
            } else if (t == 4) {
                tm = halfwave_max(tm) * c;
                up = tm > mq + CK_TAU;
                mn = up ? tm : mq;
                alpha = up ? __builtin_amdgcn_exp2f(mq - mn) : 1.0f;
                m[qs] = mn;
            } else if (t < 13) {
                // v_exp_f32 of arguments <= 8; results below 2^-126 flush to 0
                const int k = t - 5;
                const float e0 = __builtin_amdgcn_exp2f(fmaf(s_in[2 * k], c, -mn));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(s_in[2 * k + 1], c, -mn));
                pw[k] = pack_bf16x2(e0, e1);
            } else if (t < 15) {
                // row sum of the bf16 weights the PV product uses
#pragma unroll
                for (int k = 4 * (t - 13); k < 4 * (t - 13) + 4; ++k)
                    lsum = __builtin_amdgcn_fdot2_f32_bf16(
                        __builtin_bit_cast(bf16x2, pw[k]),
                        __builtin_bit_cast(bf16x2, 0x3F803F80u), lsum, false);
            } else {
                l[qs] = FRESH ? lsum : l[qs] * alpha + lsum;
                asm volatile("" : "+v"(l[qs]));
                pout[0] = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
                pout[1] = as_bf16x8(u32x4{pw[4], pw[5], pw[6], pw[7]});
            }
            ld(t);
            ext(t);
            __builtin_amdgcn_sched_barrier(0);
        }
        return up;
    };
    auto rescale = [&](int qb, float alpha) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[qb][db][i] *= alpha;
    };
    using I0 = std::integral_constant<int, 0>;
    using IK = std::integral_constant<int, KS>;
    using I8 = std::integral_constant<int, 8>;
    using BT = std::true_type;
    using BF = std::false_type;
    auto none = [](int) {};
    // store work of the previous tile's block qb: its O pieces and (m, l)
    // over slots 0 .. 8 of a phase
    auto store_ext = [&](int qb, int64_t q0p, float mp, float lp) {
        return [&, qb, q0p, mp, lp](int t) {
            const int64_t blk = part_blk + (q0p >> 5) + qb;
            if (t < 8) store_partial_piece(p, blk, o[qb], t, lane);
            if (t == 8) store_partial_ml(p, bh, chunk, q0p + 32 * qb + l32, mp, halfwave_sum(lp));
        };
    };

    for (int i = 0; i < ntiles; ++i) {
        const int64_t q0 = tile_q0(i);
        const int64_t q0p = i > 0 ? tile_q0(i - 1) : q0;
        const int64_t qnx = tile_q0(i + 1);  // rows past Q are clamped to q0
        float a0 = 1.0f, a1 = 1.0f;
        // X(0): previous tile's O1 += PV(V_7); store its block 0
        {
            const float mp = m[0], lp = l[0];
            auto ld = [&](int t) { if (t < KS) kb[1][t] = lds_k(1, t); };
            phase(IK{}, I8{}, BF{}, BT{}, kb[0], qf[1], s1, vb[1], 1, p1, 0, s0, p0, a0, ld,
                  store_ext(0, q0p, mp, lp));
        }
        // Y(0): O0 = PV(V_0) from zero; store the previous tile's block 1
        {
            const float mp = m[1], lp = l[1];
            auto ld = [&](int t) { if (t < 8) vb[1][t >> 2][t & 3] = lds_v(1, t); };
            phase(IK{}, I8{}, BT{}, BT{}, kb[1], qf[0], s0, vb[0], 0, p0, 1, s1, p1, a1, ld,
                  store_ext(1, q0p, mp, lp));
        }
        // X(1): O1 = PV(V_0) from zero
        {
            auto ld = [&](int t) { if (t < KS) kb[0][t] = lds_k(2, t); };
            const bool up = phase(IK{}, I8{}, BT{}, BF{}, kb[1], qf[1], s1, vb[0], 1, p1, 0, s0,
                                  p0, a0, ld, none);
            if (__any(up)) rescale(0, a0);
        }
        // Y(1)
        {
            auto ld = [&](int t) { if (t < 8) vb[0][t >> 2][t & 3] = lds_v(2, t); };
            const bool up = phase(IK{}, I8{}, BF{}, BF{}, kb[0], qf[0], s0, vb[1], 0, p0, 1, s1,
                                  p1, a1, ld, none);
            if (__any(up)) rescale(1, a1);
        }
#pragma unroll
        for (int j = 2; j < NSTEP; ++j) {
            const int cj = j & 1, nj = cj ^ 1;
            const int jn = (j + 1) % NSTEP;  // next step (the next tile's first after the last)
            // X(j); the next tile's queries are requested during X(4) / X(5)
            {
                auto ld = [&](int t) { if (t < KS) kb[nj][t] = lds_k(jn, t); };
                auto ext = [&](int t) {
                    if (j == 4 && t == 0) load_q_block<DK>(qn[0], p, b, h, qnx, q0, lane);
                    if (j == 5 && t == 0) load_q_block<DK>(qn[1], p, b, h, qnx + 32, q0, lane);
                };
                const bool up = phase(IK{}, I8{}, BF{}, BF{}, kb[cj], qf[1], s1, vb[nj], 1, p1,
                                      0, s0, p0, a0, ld, ext);
                if (__any(up)) rescale(0, a0);
            }
            // Y(j); Y(7) scores the next tile's first step with its block-0 queries
            {
                auto ld = [&](int t) { if (t < 8) vb[nj][t >> 2][t & 3] = lds_v(jn, t); };
                const bool up = phase(IK{}, I8{}, BF{}, BF{}, kb[nj], j + 1 < NSTEP ? qf[0] : qn[0],
                                      s0, vb[cj], 0, p0, 1, s1, p1, a1, ld, none);
                if (__any(up)) rescale(1, a1);
            }
        }
        // the next tile's queries become this tile's
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) qf[qb][kk] = qn[qb][kk];
    }
    // the last tile: O1 += PV(V_7), then both partials
#pragma unroll
    for (int ts = 0; ts < 2; ++ts)
#pragma unroll
        for (int db = 0; db < 4; ++db) o[1][db] = mfma32(vb[1][ts][db], p1[ts], o[1][db]);
    const int64_t q0l = tile_q0(ntiles - 1);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
        store_partial(p, bh, chunk, q0l + 32 * qb, o[qb], m[qb], halfwave_sum(l[qb]), lane);
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
        // The chunk's center ids and this head's biases are loaded and
        // published to LDS once V's first decode stages are in flight, so
        // that the latencies of both overlap.
        auto publish = [&]() {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const ChunkCodec& cd = p.codec[cc];
                int id = 0;
                if (cd.centers && t < valid) {
                    // ids outside the table are clamped so that a corrupt
                    // payload cannot read out of bounds (valid payloads never
                    // hold them)
                    const int64_t key = tok0 + t;
                    id = read_id(cd.ids, cd.id_bytes, (int64_t)b * p.N + history_row(p, key));
                    id = min(max(id, 0), cd.num_centers - 1);
                }
                sm.ids[cc][t] = id;
                const int width = cc == 0 ? DK : CK_D;
                if (t < width)
                    sm.bias[cc][t] =
                        cd.bias ? bf16_round(cd.bias[(int64_t)h * cd.bias_hs + t]) : 0.0f;
            }
            __syncthreads();
        };
        auto nothing = []() {};
        // V first: its decoder slices are staged in the (not yet written)
        // V^T region and its centers in the K region; then K, with its
        // slices staged in the K region once V's epilogue is done.
        uint16_t* vt_scratch = &sm.vt[0][0];
        uint16_t* k_scratch = &sm.k[0][0];
        if (p.codec[1].centers)
            decode_codec<1, true, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                              wave, lane, publish);
        else
            decode_codec<1, false, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                               wave, lane, publish);
        __syncthreads();
        if (p.codec[0].centers)
            decode_codec<0, true, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid, wave,
                                            lane, nothing);
        else
            decode_codec<0, false, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid,
                                             wave, lane, nothing);
    } else if (DK == CK_D) {
        load_current_chunk(sm, p, b, h, tok0, valid, t);
    }
    __syncthreads();

    const int nsub = (valid + 31) / 32;
    const int nqt = (int)cdiv(p.Q, CK_QT);
    constexpr int WAVES = CK_THREADS / 64;
    if (valid == CK_T) {
        // full chunk: the wave's two-block tiles (wave + 4 i, those with
        // q0 + 32 < Q: a prefix of its tiles) as one pipeline, then at most
        // one single-block tile
        const int t2 = p.Q > 32 ? (int)((p.Q + 31) / CK_QT) : 0;
        const int n2 = t2 > wave ? (t2 - wave + WAVES - 1) / WAVES : 0;
        if (n2 > 0) attend_stream<DK>(sm, p, b, h, bh, chunk, wave, lane, n2);
        const int qt = wave + WAVES * n2;
        if (qt < nqt) {
            const int64_t q0 = (int64_t)qt * CK_QT;
            bf16x8 qf[2][8];
            load_q_block<DK>(qf[0], p, b, h, q0, q0, lane);
            attend_qtile<DK, 1, true>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q0);
        }
        return;
    }
    bf16x8 qf[2][8];
    if (wave < nqt) {
        load_q_block<DK>(qf[0], p, b, h, (int64_t)wave * CK_QT, (int64_t)wave * CK_QT, lane);
        load_q_block<DK>(qf[1], p, b, h, (int64_t)wave * CK_QT + 32, (int64_t)wave * CK_QT, lane);
    }
    for (int qt = wave; qt < nqt; qt += WAVES) {
        const int64_t q0 = (int64_t)qt * CK_QT;
        // the wave's next tile, or this one again (a harmless in-bounds reload)
        const int64_t q_next = qt + WAVES < nqt ? q0 + WAVES * CK_QT : q0;
        if (q0 + 32 >= p.Q)
            attend_qtile<DK, 1, false>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
        else
            attend_qtile<DK, 2, false>(sm, p, b, h, bh, chunk, q0, nsub, valid, lane, qf, q_next);
    }
}

// Merge the chunk partials of every (b, h, q).  A 256-thread block owns one
// 32-query block; its four waves take every fourth chunk, each lane reading
// the lane-order payload the attention wave stored, and sum through LDS.
// out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c (O_c unnormalised); no chunks give
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
    const u32x2* ml = reinterpret_cast<const u32x2*>(p.part_ml) + bh * NC * lse_stride + qi;
    // the largest running max; eight independent maxima keep eight loads in flight
    float mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mx[e] = -INFINITY;
    int cc0 = 0;
    for (; cc0 + 8 <= NC; cc0 += 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            mx[e] = fmaxf(mx[e], __uint_as_float(ml[(cc0 + e) * lse_stride][0]));
    }
    for (; cc0 < NC; ++cc0) mx[0] = fmaxf(mx[0], __uint_as_float(ml[cc0 * lse_stride][0]));
    float M = mx[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) M = fmaxf(M, mx[e]);
    const float Mu = M == -INFINITY ? 0.0f : M;
    // out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c (O_c unnormalised)
    float L = 0.0f, acc[64];
#pragma unroll
    for (int e = 0; e < 64; ++e) acc[e] = 0.0f;
    const uint16_t* src = p.part_o + (bh * NC * p.qblocks + qblk) * 4096 + lane * 8;
    const int64_t cstride = (int64_t)p.qblocks * 4096;
#pragma unroll 2
    for (int cc = wave; cc < NC; cc += CB_WAVES) {
        const u32x2 mlc = ml[cc * lse_stride];
        const float wt = exp2f(__uint_as_float(mlc[0]) - Mu);
        L += wt * __uint_as_float(mlc[1]);
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
    return blocks * 32 * CK_D * sizeof(uint16_t) + blocks * 32 * 2 * sizeof(float);
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
    p.part_ml = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) +
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
