// nkv_chunk.hip -- decode-once schedules of nkv_attend for gfx950
// (NKV_SCHEDULE_KEY_CHUNKS).
//
// Two schedules live here; both decode every history key once per head.
//  - The staged schedule (the drtile / stage8 decode, tile_xform_kernel,
//    flash8_kernel and staged_combine_kernel, further below) serves every
//    call at K/Q width 128 and the reader widths 32/64 with ranks up to the
//    resident decoder's 384: the decode writes each 128-key tile once into
//    the call's workspace, in the flash kernel's LDS layout, and the flash
//    kernel streams the tiles back with O held in registers over a whole
//    key split.
//  - The key-chunk kernel (chunk8_kernel, next) serves reader widths 32/64
//    with ranks above 384: the decoded K/V stay in LDS, and each (chunk,
//    query block) leaves a partial.
//
// Key-chunk kernel: a 512-thread block (8 waves, two per SIMD) owns one (batch, head, chunk)
// of 256 keys.  It decodes the chunk's K and V once into LDS -- K[key][d]
// and V^T[d][key], bf16, 137 KB -- and then every wave attends its share of
// ALL the head's 32-query blocks to those keys.  Each (query, chunk) leaves
// a partial: the chunk-local O (bf16, unnormalised) with its running max and
// row sum.  A combine kernel merges the partials of every query by
// log-sum-exp (CN/core.py:33-42 applied over all chunks).  A 32-query
// block's partial is stored in the MFMA accumulator's lane order (8 KB:
// eight 1 KB rows of 16 bytes per lane), so the stores here and the
// combine's loads are contiguous.
// Decoding each history key once per head, instead of once per query tile,
// removes the decode GEMM's re-execution; the price is the partial traffic
// (256 + 8 bytes per query and chunk).
//
// Decode (per wave: 32 keys of the chunk, both codecs; MFMA 32x32x16 bf16):
//   K^T = W_K[h*128 + d, :] . Z^T   (A = decoder rows, B = unpacked codes)
//   V   = Z . W_V[h*128 + d, :]^T   (A = unpacked codes, B = decoder rows)
// The k (rank) axis is walked in blocks of 64: lane half hf supplies
// k = 64*kq + 32*hf + 8*j + [0, 8) at step j of block kq.  That permutation of
// the summation index is applied to both operands, so one 16-byte load per
// lane fetches the packed codes of four MFMA steps, and they share one scale
// group (group % 32 == 0).  Decoder rows stream through an LDS ring (see
// below).  The epilogue is the reference decode arithmetic
// bf16(bf16(acc + bf16(mean)) + center[id]) (MG:438-454); the accumulator
// orientation puts four consecutive d (K) or four consecutive keys (V) in
// one lane, so both tiles are written with 8-byte LDS stores.
// Current-chunk keys (uncompressed bf16) are copied instead of decoded.
//
// Attention (per wave and 32-query block; queries on the MFMA column axis):
//   S^T = K Q^T, P = exp2(S * c - m), O^T += V^T P^T
// over eight 32-key steps.  The running max is raised only when a score
// exceeds it by more than 2^8 (P <= 256 otherwise), so O is rarely rescaled.
#include "nkv_camera.h"
#include "nkv_common.h"
#include "nkv_internal.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <type_traits>
#include <vector>

namespace nkv {

// The key-chunk kernel's partials are written non-temporally: they are read
// once, by the combine, after the chunk kernel has written all of them
// (hundreds of MB at long histories), so caching them only evicts the codec
// tables and decoded tiles that the running blocks re-read.  Plain stores measured 7 % slower over
// the whole call at 1,560 queries x 14,040 keys (0.580 vs 0.540 ms), and
// head-group launches sized for the partials to stay in the MALL slower
// still (0.547-0.573 ms; at 50,700 keys 1.55 vs 1.02 ms).
#define NT_STORE(v, ptr) __builtin_nontemporal_store((v), (ptr))

constexpr int CK_T = 256;        // keys per chunk
constexpr int CK_CUR_SPLITS = 3; // most blocks per current-key chunk (query shares)
constexpr int CK_D = 128;        // head dim
constexpr int CK_KROW = CK_D + 8;   // K row: 68 dwords (b128 reads conflict-free)
constexpr float CK_TAU = 8.0f;   // lazy-rescale threshold (log2 units)

// K tile row pitch for a K/Q width DK (b128 reads of 8 rows hit distinct banks)
template <int DK>
struct KTile {
    static constexpr int ROW = DK + 8;
};

struct ChunkParams {
    int B, H;           // H: heads of this launch (launch head i)
    int nch_hist, nch_total;
    int qblocks;        // 32-query blocks per (b, i): cdiv(Q, 32)
    int cur_splits;     // blocks per current-key chunk, each attending a share of the query blocks
    int64_t Q;
    int64_t N;          // history tokens per batch item in the codec arrays
    int64_t n_rows;     // history keys attended
    const int32_t* rows;  // [n_rows] codec rows of those keys, or null: rows 0 .. n_rows-1
    int64_t Nc;
    float scale_log2;
    const uint16_t* q;  // [B, Q, H, DK] (strides)
    int64_t q_sb, q_st, q_sh;
    const int32_t* q_heads;  // query head of launch head i (null: i), clamped to [0, q_heads_n)
    int q_heads_n;
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
    RopeDev rope;       // RoPE of the history keys (cs_t null: none)
    CameraDev cam;      // camera P^-1 of the history keys and values (mats null: none)
    const uint32_t* cur_mask;  // visibility of the current keys per query group, or null
    const int32_t* q_group;
    int n_groups, mask_words;
    int64_t blk_base;   // first work item of this launch (blockIdx.x + blk_base)
    // staged schedule: tile images [B*H, ntiles, K / V^T image] (history
    // tiles 0 .. ntiles_hist, two per 256-key chunk, then the current keys'),
    // qpt query blocks per flash block, `splits` key ranges per query block
    uint16_t* tiles;
    int ntiles_hist, ntiles, qpt, splits, qtiles;
};

// ------------------------------------------------ multi-partition launches
// One launch of the staged schedule runs the blocks of up to NKV_MAX_PARTS
// attention partitions (the native partition and the reader groups of a
// NanoKV-Fast call, or one nkv_attend call), each with its own ChunkParams
// and K/Q width.  Blocks [seg_first[s], seg_first[s + 1]) run segment s: work
// seg_kind[s] of partition seg_part[s] (seg_ranges[s]: the block count of a
// decode segment, one range of its history tiles per block).
constexpr int MP_SEGS = 4 * NKV_MAX_PARTS;
enum : int { SEG_K = 0, SEG_V = 1, SEG_CUR = 2, SEG_FLASH = 3, SEG_XFORM = 4, SEG_TABLE = 5 };
struct MultiParams {
    ChunkParams part[NKV_MAX_PARTS];
    int dk[NKV_MAX_PARTS];
    // combine: layer head of head i of partition j >= 1 (partition 0 covers
    // every head of the layer and holds its output)
    const int32_t* heads[NKV_MAX_PARTS];
    int nparts, nseg;
    int seg_part[MP_SEGS], seg_kind[MP_SEGS], seg_ranges[MP_SEGS];
    int64_t seg_first[MP_SEGS + 1];
};

// Segment of block x (a scan over the uniform table).
__device__ __forceinline__ int multi_segment(const MultiParams& P, int64_t x) {
    int sg = 0;
#pragma unroll
    for (int i = 1; i < MP_SEGS; ++i)
        if (i < P.nseg && x >= P.seg_first[i]) sg = i;
    return sg;
}

// Codec row of attended history key `key`; rows outside the codec are
// clamped so that a bad row list cannot read out of bounds.
__device__ __forceinline__ int64_t history_row(const ChunkParams& p, int64_t key) {
    if (!p.rows) return key;
    return min(max((int64_t)p.rows[key], (int64_t)0), p.N - 1);
}

// ------------------------------------------------------------------ decode
// Decoder slices W[row d of the launch head][64*s, +64) (WIDTH rows of 128
// bytes) stream into a ring of DS_NBUF LDS buffers by direct-to-LDS loads
// (global_load_lds_dwordx4: no register staging), DS_AHEAD slices ahead of
// the MFMAs.  The block's waves each copy a share of every slice, so every
// decoder element is fetched from L2 once per block.  Rows are stored
// unpadded with their 16-byte chunks XOR-swizzled: chunk c of row r sits at
// chunk c ^ ((r >> 1) & 7).  gfx950 serves 16-byte LDS reads 16 lanes at a
// time over 64 banks; with 128-byte rows, rows r and r + 1 share a bank half
// only if their chunks differ, so the MFMA operand reads of 16 consecutive
// rows are conflict-free, while every load instruction still fills one
// contiguous 1 KB of LDS.
//
// A stage (slice s) = its decoder rows plus this wave's codes and scales of
// slice s, which go to a register ring of DS_AHEAD entries.  Loads complete
// in issue order, so waiting for stage s is one vmcnt bound: the stages
// issued after it may stay in flight.
constexpr int DS_NBUF = 4;
constexpr int DS_AHEAD = 3;
// The rings fit in the regions that hold no live data while they are used:
// V's decode stages in the V^T region, K's in the K region; V's centers are
// staged in the K region.
static_assert(DS_NBUF * CK_D * 64 <= CK_T * CK_KROW, "decoder staging must fit in the K region");
static_assert(CK_T * CK_D <= CK_T * CK_KROW, "V centers are staged in the K region");


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
    const int hq = p.q_heads ? min(max(ldg(p.q_heads + h), 0), p.q_heads_n - 1) : h;
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (qi < p.Q ? qi : q_safe) * p.q_st +
                           (int64_t)hq * p.q_sh + W::HALF * hf;
#pragma unroll
    for (int kk = 0; kk < W::KSTEPS; ++kk)
        qf[kk] = as_bf16x8(*reinterpret_cast<const u32x4*>(qrow + W::block(kk)));
}

// The partial of one 32-query block for this chunk: its O (unnormalised,
// bf16) and per query the running max m (log2 units) and row sum l, so that
// the combine forms sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.  Lane
// dword k of the block holds o[db = k/8][2*(k%8) + {0, 1}] and is stored at
// 1 KB * (k/4) + 16 B * lane + 4 B * (k%4): every store instruction writes
// 1 KB contiguous.  Query columns past Q hold finite values that the combine
// ignores; both half-waves store the same (m, l) of their query.
// NT: non-temporal stores (the key-chunk kernel's partials, see NT_STORE);
// the staged flash kernel's few partials (30 MB at cfg1) are stored plainly,
// which its combine reads about 1 us faster.
template <bool NT>
__device__ __forceinline__ void store_partial_piece(const ChunkParams& p, int64_t blk,
                                                    const f32x16 (&o)[4], int st, int lane) {
    uint16_t* dst = p.part_o + blk * 4096 + lane * 8;
    const int db = st >> 1, i0 = 8 * (st & 1);
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(o[db][i0 + 2 * e], o[db][i0 + 2 * e + 1]);
    if (NT) NT_STORE(w, reinterpret_cast<u32x4*>(dst + 512 * st));
    else *reinterpret_cast<u32x4*>(dst + 512 * st) = w;
}

template <bool NT>
__device__ __forceinline__ void store_partial_ml(const ChunkParams& p, int64_t bh, int chunk,
                                                 int64_t qcol, float m, float lt) {
    const int64_t idx = (bh * p.nch_total + chunk) * ((int64_t)p.qblocks * 32) + qcol;
    const u32x2 v{__float_as_uint(m), __float_as_uint(lt)};
    if (NT) NT_STORE(v, reinterpret_cast<u32x2*>(p.part_ml + 2 * idx));
    else *reinterpret_cast<u32x2*>(p.part_ml + 2 * idx) = v;
}

template <bool NT = true>
__device__ __forceinline__ void store_partial(const ChunkParams& p, int64_t bh, int chunk,
                                              int64_t qblk0, const f32x16 (&o)[4], float m,
                                              float lt, int lane) {
    const int64_t blk = ((int64_t)bh * p.nch_total + chunk) * p.qblocks + (qblk0 >> 5);
#pragma unroll
    for (int st = 0; st < 8; ++st) store_partial_piece<NT>(p, blk, o, st, lane);
    store_partial_ml<NT>(p, bh, chunk, qblk0 + (lane & 31), m, lt);
}

// ======================================================= 8-wave key-chunk kernel
// The same key-chunk schedule with eight waves per block, two per SIMD: while
// one wave runs VALU work (INT4 unpack, decode epilogue, softmax) the other's
// MFMAs keep the matrix core busy, so each wave's own code can stay serial.
// Each wave decodes 32 of the chunk's keys and attends 32-query blocks.
// Every attention operand is one 16-byte LDS read (gfx950 serves those at
// up to ~190 B/clk per CU with several waves per SIMD, against ~125 for
// 8-byte reads).
constexpr int C8_THREADS = 512;
constexpr int C8_WAVES = C8_THREADS / 64;
constexpr int C8_VROW = CK_T + 8;  // V^T row: 132 dwords, 16 rows of b128 reads hit distinct banks

typedef short short4v __attribute__((ext_vector_type(4)));

struct Chunk8Smem {
    uint16_t k[CK_T][CK_KROW];  // K tile (also decoder-slice and center staging)
    uint16_t vt[CK_D][C8_VROW];  // V^T[d][vt_col(key)]
    const uint16_t* crow[2][CK_T];  // center row of each key (the launch head's columns)
    float bias[2][CK_D];
};
static_assert(sizeof(Chunk8Smem) <= 160 * 1024, "LDS budget");
static_assert(DS_NBUF * CK_D * 64 <= CK_D * C8_VROW, "decoder staging must fit in the V^T region");

// V^T column of a key: inside each group of 16 keys the middle two quarters
// swap (0 1 2 3 -> 0 2 1 3), so the eight keys one lane half supplies to a
// PV MFMA step (quarters hf and hf + 2 of the group) are one contiguous
// 16-byte run.
__device__ __forceinline__ int vt_col(int key) {
    const int q = (key >> 2) & 3;
    const int pq = (q == 1 || q == 2) ? 3 - q : q;
    return (key & ~15) | (pq << 2) | (key & 3);
}

// The V center rows of the wave's 32 keys, copied into LDS rows [key][128]
// (unpadded) by 8 direct-to-LDS loads of 4 rows each.
__device__ __forceinline__ void dma_v_centers8(uint16_t* vcen, const Chunk8Smem& sm, int wave,
                                               int lane) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int t = 32 * wave + 4 * e + (lane >> 4);
        __builtin_amdgcn_global_load_lds(sm.crow[1][t] + 8 * (lane & 15),
                                         NKV_LDS(vcen + (32 * wave + 4 * e) * CK_D), 16, 0, 0);
    }
}

// The DK K-center values of the wave's 32 keys as coalesced 16-byte pieces:
// entry e of lane L is piece q = 64*e + L, key 32*wave + q / (DK/8), columns
// 8 * (q % (DK/8)).
template <int DK>
__device__ __forceinline__ void load_k_center_rows8(u32x4 (&v)[DK / 16], const Chunk8Smem& sm,
                                                    int wave, int lane) {
    constexpr int PR = DK / 8;
#pragma unroll
    for (int e = 0; e < DK / 16; ++e) {
        const int q = 64 * e + lane;
        v[e] = ldg(reinterpret_cast<const u32x4*>(sm.crow[0][32 * wave + q / PR] + 8 * (q % PR)));
    }
}

// Decode this wave's 32 keys (32*wave + [0, 32) of the chunk) of codec CODEC
// to WIDTH columns: V into V^T (permuted columns), K into the K tile.  The
// decoder-slice ring and code/scale ring are those of decode_codec; each of
// the eight waves copies WIDTH/64 KB of every slice (for WIDTH = 32 waves
// 4-7 repeat waves 0-3's pieces: the same bytes to the same place).
// Read-time RoPE of the wave's 32 decoded keys in the K tile (after their
// bias and centers): lane half hf rotates pairs [WIDTH/4 * hf, +WIDTH/4) of key
// 32 * wave + l32 at the position of its codec row.  The wave's LDS
// operations stay in order, so no barrier separates this from the epilogue.
template <int WIDTH, int KROW>
__device__ __forceinline__ void rope_k_rows(uint16_t* ktile, const ChunkParams& p, int h,
                                            int64_t tok0, int valid, int wave, int lane) {
    constexpr int HP = WIDTH / 4;  // pairs per lane
    const int hf = lane >> 5, kt = 32 * wave + (lane & 31);
    const RopeRows rr = rope_rows(p.rope, history_row(p, tok0 + (kt < valid ? kt : 0)));
    uint16_t* krow = ktile + kt * KROW + 2 * HP * hf;
    const int32_t* pmap = p.rope.pairs ? p.rope.pairs + (int64_t)h * (WIDTH / 2) + HP * hf
                                       : nullptr;
    // every table load of the lane is issued before the first rotation (the
    // decode's accumulators are dead here), so their latencies overlap
    double2 cs[HP];
#pragma unroll
    for (int e = 0; e < HP; ++e) {
        const int pj = pmap ? pmap[e] : HP * hf + e;
        const f64x2 v = ldg(reinterpret_cast<const f64x2*>(rope_entry(p.rope, rr, pj)));
        cs[e] = double2{v.x, v.y};
    }
#pragma unroll
    for (int q = 0; q < HP / 4; ++q) {
        const u32x4 kv = *reinterpret_cast<const u32x4*>(krow + 8 * q);
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = rope_pair(kv[e], cs[4 * q + e].x, cs[4 * q + e].y);
        *reinterpret_cast<u32x4*>(krow + 8 * q) = y;
    }
}

// Camera P^-1 of the wave's 32 decoded keys (after RoPE) in the K tile: the
// two lane halves share key 32 * wave + l32.  Full-width keys use the
// camera's layout; reader keys (WIDTH < 128, or a block map) the launch
// head's sub-frame of each 8-dim block.
template <int WIDTH, int KROW>
__device__ __forceinline__ void camera_k_rows(uint16_t* ktile, const ChunkParams& p, int b, int h,
                                              int64_t tok0, int valid, int wave, int lane) {
    const int hf = lane >> 5, kt = 32 * wave + (lane & 31);
    const float* M = camera_mats(p.cam, b, history_row(p, tok0 + (kt < valid ? kt : 0)));
    uint16_t* krow = ktile + kt * KROW;
    auto get = [&](int d) { return bf16_bits_to_f32(krow[d]); };
    auto put = [&](int d, float y) { krow[d] = f32_to_bf16_bits(y); };
    if (p.cam.blocks)
        camera_row_blocks<WIDTH>(M, p.cam.blocks + (int64_t)h * (WIDTH / 8), hf, get, put);
    else if (WIDTH == CK_D)
        camera_row<CK_D>(M, p.cam.layout, hf, get, put);
}

template <int CODEC, bool HAS_C, int WIDTH, int KROW, typename Pre>
__device__ __forceinline__ void decode_codec8(Chunk8Smem& sm, uint16_t* wst, const ChunkCodec& c,
                                              const ChunkParams& p, int b, int h, int64_t tok0,
                                              int valid, int wave, int lane, Pre&& pre) {
    constexpr int NDT = WIDTH / 32;
    constexpr int PIECES = WIDTH / 8;                        // 1 KB pieces per slice
    constexpr int LPW = PIECES >= C8_WAVES ? PIECES / C8_WAVES : 1;
    constexpr int STAGE = LPW + 2;                           // vm instructions per stage
    constexpr int SLICE = WIDTH * 64;
    const int hf = lane >> 5, l32 = lane & 31;
    const int R = c.r, KQ = R >> 6, G = c.group;
    const bool f16 = c.scale_dtype == NKV_DTYPE_FP16;
    const int tl = 32 * wave + l32;
    // keys past the chunk end decode key 0's codes (finite, never attended)
    const uint8_t* prow;
    const uint16_t* srow;
    codec_row_ptrs(c, b, p.N, history_row(p, tok0 + (tl < valid ? tl : 0)), prow, srow);
    prow += 16 * hf;
    // slice pieces: lane L of piece q brings logical chunk
    // (L % 8) ^ ((row >> 1) & 7) of row 8 q + L / 8
    const int piece_row = lane >> 3;
    const uint16_t* wsrc = c.w + (int64_t)h * c.w_hs + (int64_t)piece_row * R;
    auto issue_slice = [&](int s) {
        uint16_t* dst = wst + (s % DS_NBUF) * SLICE;
#pragma unroll
        for (int e = 0; e < LPW; ++e) {
            const int piece = (LPW * wave + e) % PIECES;
            const int chunk = (lane & 7) ^ ((4 * (piece & 1) + (piece_row >> 1)) & 7);
            __builtin_amdgcn_global_load_lds(wsrc + (int64_t)8 * piece * R + 64 * s + 8 * chunk,
                                             NKV_LDS(dst + piece * 512), 16, 0, 0);
        }
    };
    auto issue_codes = [&](int s, u32x4& pk, uint16_t& sb) {
        pk = ldg(reinterpret_cast<const u32x4*>(prow + 32 * s));
        sb = ldg(srow + (64 * s + 32 * hf) / G);
    };

    f32x16 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x16{};

    uint16_t* vcen = &sm.k[0][0];
    u32x4 kcen[WIDTH / 16];
    if (CODEC == 0 && HAS_C) load_k_center_rows8<WIDTH>(kcen, sm, wave, lane);
    u32x4 pk[DS_AHEAD];
    uint16_t sc[DS_AHEAD];
#pragma unroll
    for (int i = 0; i < DS_AHEAD; ++i)
        if (i < KQ) {
            issue_slice(i);
            issue_codes(i, pk[i], sc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    pre();
    constexpr int NVC = CODEC == 1 && HAS_C ? 8 : 0;
    if (CODEC == 1 && HAS_C) dma_v_centers8(vcen, sm, wave, lane);
    __builtin_amdgcn_sched_barrier(0);

    int wofs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wofs[j] = l32 * 64 + 8 * ((4 * hf + j) ^ ((l32 >> 1) & 7));

    u32x4 zc;
    float scl = 0.0f, ns7 = 0.0f;
    if (KQ > 0) {
        scl = f16 ? f16_bits_to_f32(sc[0]) : bf16_bits_to_f32(sc[0]);
        ns7 = -7.0f * scl;
        Unpack8 u;
        u.split(pk[0][0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) zc[e] = u.pair(e, scl, ns7);
    }
    for (int s0 = 0; s0 < KQ; s0 += DS_AHEAD) {
#pragma unroll
        for (int i = 0; i < DS_AHEAD; ++i) {
            const int s = s0 + i;
            if (s >= KQ) break;
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
            // sub-step j+1's codes (for the last, the next slice's first) are
            // unpacked under sub-step j's MFMAs, a pair of codes per slot
            const int inx = (i + 1) % DS_AHEAD;
            const float scn = f16 ? f16_bits_to_f32(sc[inx]) : bf16_bits_to_f32(sc[inx]);
            const float nsn = -7.0f * scn;
            u32x4 zn;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bf16x8 w[NDT];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) w[dt] = lds_b128(wb + 32 * dt * 64 + wofs[j]);
                Unpack8 u;
                u.split(j + 1 < 4 ? pk[i][j + 1] : pk[inx][0]);
#pragma unroll
                for (int m = 0; m < NDT; ++m) {
                    acc[m] = CODEC == 0 ? mfma32(w[m], as_bf16x8(zc), acc[m])
                                        : mfma32(as_bf16x8(zc), w[m], acc[m]);
#pragma unroll
                    for (int q = (4 * m) / NDT; q < (4 * (m + 1)) / NDT; ++q) {
                        zn[q] = j + 1 < 4 ? u.pair(q, scl, ns7) : u.pair(q, scn, nsn);
                        if (j + 1 == 4) asm volatile("" : "+v"(zn[q]));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                zc = zn;
            }
            scl = scn;
            ns7 = nsn;
            __builtin_amdgcn_sched_barrier(0);
            if (s + DS_AHEAD < KQ) issue_codes(s + DS_AHEAD, pk[i], sc[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();

    if (CODEC == 0) {
        // acc[dt] element i: d = 32*dt + 8*(i/4) + 4*hf + i%4, key 32*wave + l32
        uint16_t* ktile = &sm.k[0][0];
        const int t = 32 * wave + l32;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * dt + 8 * g + 4 * hf;
                float a[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) a[e] = acc[dt][4 * g + e] + sm.bias[0][d + e];
                const u32x2 r = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
                *reinterpret_cast<u32x2*>(ktile + t * KROW + d) = r;
            }
        if (HAS_C) {
            // the wave's own rows: its LDS operations stay in order
            constexpr int PR = WIDTH / 8;
#pragma unroll
            for (int e = 0; e < WIDTH / 16; ++e) {
                const int q = 64 * e + lane;
                u32x4* slot = reinterpret_cast<u32x4*>(ktile + (32 * wave + q / PR) * KROW +
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
        if (rope_on(p.rope)) rope_k_rows<WIDTH, KROW>(ktile, p, h, tok0, valid, wave, lane);
        if (p.cam.mats) camera_k_rows<WIDTH, KROW>(ktile, p, b, h, tok0, valid, wave, lane);
    } else {
        // acc[dt] element i: key 32*wave + 8*(i/4) + 4*hf + i%4, d = 32*dt + l32.
        // The centers of keys t0 .. t0+3 at column d come from one LDS
        // transpose read (ds_read_b64_tr_b16): within a group of 16 lanes,
        // lane j receives element j % 4 of the 8-byte rows that lanes
        // j / 4, j / 4 + 4, j / 4 + 8, j / 4 + 12 address, so lane x = a + 4k
        // addresses key t0 + k at columns dbase + 4a .. +4 and lane j gets
        // the four keys at column dbase + j.
        const int tr_x = lane & 15;
        const int tr_off = (tr_x >> 2) * CK_D + 4 * (tr_x & 3) + 16 * ((lane >> 4) & 1);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t0 = 32 * wave + 8 * g + 4 * hf;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int d = 32 * dt + l32;
                const float bias = sm.bias[1][d];
                short4v cen = {};
                if (HAS_C)
                    cen = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) short4v*)(vcen + t0 * CK_D + 32 * dt + tr_off));
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = bf16_round(acc[dt][4 * g + e] + bias);
                    v[e] = HAS_C ? a + __uint_as_float((uint32_t)(uint16_t)cen[e] << 16) : a;
                }
                const u32x2 r = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                *reinterpret_cast<u32x2*>(&sm.vt[d][vt_col(t0)]) = r;
            }
        }
        if (p.cam.mats) {
            // camera P^-1 of the wave's 32 value columns of V^T: the two lane
            // halves share key 32 * wave + l32
            const int kt = 32 * wave + l32;
            const float* M = camera_mats(p.cam, b, history_row(p, tok0 + (kt < valid ? kt : 0)));
            const int col = vt_col(kt);
            camera_row<CK_D>(
                M, p.cam.layout, hf, [&](int d) { return bf16_bits_to_f32(sm.vt[d][col]); },
                [&](int d, float y) { sm.vt[d][col] = f32_to_bf16_bits(y); });
        }
    }
}

// Current (uncompressed) keys of this chunk into the K tile and V^T (DK =
// 128).  Thread t handles keys 4*(t % 64) .. +4 and d = 16*(t / 64) .. +16:
// K rows go out as 16-byte stores, V^T as one 8-byte store (four keys) per
// d.  Keys past `valid` are zero.
__device__ __forceinline__ void load_current_chunk8(Chunk8Smem& sm, const ChunkParams& p, int b,
                                                    int h, int64_t tok0, int valid, int t) {
    const int k0 = 4 * (t & 63), d0 = 16 * (t >> 6);
    u32x4 kv[4][2], vv[4][2];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int key = k0 + e;
        const bool ok = key < valid;
        const int64_t tok = tok0 + (ok ? key : 0);
        const uint16_t* ks = p.k_cur + (int64_t)b * p.k_sb + tok * p.k_st + (int64_t)h * p.k_sh + d0;
        const uint16_t* vs = p.v_cur + (int64_t)b * p.v_sb + tok * p.v_st + (int64_t)h * p.v_sh + d0;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            kv[e][x] = ok ? *reinterpret_cast<const u32x4*>(ks + 8 * x) : u32x4{0, 0, 0, 0};
            vv[e][x] = ok ? *reinterpret_cast<const u32x4*>(vs + 8 * x) : u32x4{0, 0, 0, 0};
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int x = 0; x < 2; ++x)
            *reinterpret_cast<u32x4*>(&sm.k[k0 + e][d0 + 8 * x]) = kv[e][x];
    const int col = vt_col(k0);
#pragma unroll
    for (int dd = 0; dd < 16; ++dd) {
        const int x = dd >> 3, w = (dd & 7) >> 1, sh = 16 * (dd & 1);
        auto val = [&](int e) { return (vv[e][x][w] >> sh) & 0xffffu; };
        *reinterpret_cast<u32x2*>(&sm.vt[d0 + dd][col]) =
            u32x2{val(0) | (val(1) << 16), val(2) | (val(3) << 16)};
    }
}

// Decode the chunk's V (into V^T) and K (into the K tile) for (b, h): every
// thread of the block takes part; the tile is complete after a barrier.
template <int DK>
__device__ __forceinline__ void fill_history8(Chunk8Smem& sm, const ChunkParams& p, int b, int h,
                                              int64_t tok0, int valid, int t, int wave,
                                              int lane) {
    constexpr int KROW = KTile<DK>::ROW;
    auto publish = [&]() {
        if (t < CK_T) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const ChunkCodec& cd = p.codec[cc];
                // keys past the chunk end take key 0's center (finite,
                // never attended)
                if (cd.has_centers)
                    sm.crow[cc][t] = center_row(cd, b, h, p.N,
                                                history_row(p, tok0 + (t < valid ? t : 0)));
                if (t < (cc == 0 ? DK : CK_D))
                    sm.bias[cc][t] =
                        cd.bias ? bf16_round(cd.bias[(int64_t)h * cd.bias_hs + t]) : 0.0f;
            }
        }
        __syncthreads();
    };
    auto nothing = []() {};
    uint16_t* vt_scratch = &sm.vt[0][0];
    uint16_t* k_scratch = &sm.k[0][0];
    if (p.codec[1].has_centers)
        decode_codec8<1, true, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                           wave, lane, publish);
    else
        decode_codec8<1, false, CK_D, KROW>(sm, vt_scratch, p.codec[1], p, b, h, tok0, valid,
                                            wave, lane, publish);
    __syncthreads();
    if (p.codec[0].has_centers)
        decode_codec8<0, true, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid,
                                         wave, lane, nothing);
    else
        decode_codec8<0, false, DK, KROW>(sm, k_scratch, p.codec[0], p, b, h, tok0, valid,
                                          wave, lane, nothing);
}

// One wave attends its 32-query blocks (wave + 8 i) to the chunk in LDS,
// key step by key step: S^T = K Q^T (KS MFMAs), online softmax, O^T += V^T
// P^T (8 MFMAs).  The next step's K and V fragments are read as soon as the
// current ones have been issued to the matrix core, and the next block's
// queries are requested during its predecessor.
// MASK: the chunk holds current keys tok0 .. (keys of the current chunk) and
// each query sees only the keys its group's bits of p.cur_mask allow; a
// query that sees no key of a step keeps m = -inf, and its exponentials use
// 0 as the reference so that they are 0, not NaN.
template <int DK, bool MASK>
__device__ __forceinline__ void attend8(const Chunk8Smem& sm, const ChunkParams& p, int b, int h,
                                        int bh, int chunk, int wave, int lane_in, int nsub,
                                        int valid, int qb_lo, int qb_hi, int64_t tok0) {
    int lane = lane_in;
    asm volatile("" : "+v"(lane));
    const int hf = lane >> 5, l32 = lane & 31;
    const float c = p.scale_log2;
    using W = DWalk<DK>;
    constexpr int KROW = KTile<DK>::ROW;
    constexpr int KS = W::KSTEPS;
    uint32_t koff = l32 * KROW + W::HALF * hf, voff = l32 * C8_VROW + 8 * hf;
    asm volatile("" : "+v"(koff));
    asm volatile("" : "+v"(voff));
    const uint16_t* kbase = &sm.k[0][0] + koff;
    const uint16_t* vbase = &sm.vt[0][0] + voff;
    auto lds_k = [&](int j, int kk) { return lds_b128(kbase + 32 * j * KROW + W::block(kk)); };
    // V^T fragment (ts, db) of step j: rows 32*db + l32, the 8 keys of half-step ts
    auto lds_v = [&](int j, int t) {
        return lds_b128(vbase + 32 * (t & 3) * C8_VROW + 32 * j + 16 * (t >> 2));
    };
    if (qb_lo + wave >= qb_hi) return;
    bf16x8 qf[KS], qn[KS], kf[KS], vf[8];
    {
        const int64_t q0 = (int64_t)(qb_lo + wave) * 32;
        load_q_block<DK>(qf, p, b, h, q0, q0, lane);
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) kf[kk] = lds_k(0, kk);
#pragma unroll
    for (int t = 0; t < 8; ++t) vf[t] = lds_v(0, t);
    const bool full = valid == CK_T;
    for (int qb = qb_lo + wave; qb < qb_hi; qb += C8_WAVES) {
        const int64_t q0 = (int64_t)qb * 32;
        // the next block's queries (rows past Q are clamped to q0); the
        // masked instance loads each block's queries when it starts instead,
        // which leaves the registers its mask needs
        if (MASK) {
            if (qb != qb_lo + wave) load_q_block<DK>(qf, p, b, h, q0, q0, lane);
        } else {
            load_q_block<DK>(qn, p, b, h, q0 + 32 * C8_WAVES, q0, lane);
        }
        const uint32_t* mrow = nullptr;
        if (MASK) {
            const int64_t qi = min(q0 + l32, p.Q - 1);
            const int g = p.q_group ? min(max(p.q_group[qi], 0), p.n_groups - 1) : 0;
            mrow = p.cur_mask + (int64_t)g * p.mask_words + (tok0 >> 5);
        }
        f32x16 o[4];
        float m = -INFINITY, l = 0.0f;
        for (int j = 0; j < nsub; ++j) {
            // wave priority is raised around each MFMA cluster: the two waves
            // of a SIMD then settle into alternation, one issuing MFMAs while
            // the other runs its softmax
            __builtin_amdgcn_s_setprio(1);
            f32x16 s = mfma32(kf[0], qf[0], f32x16{});
#pragma unroll
            for (int kk = 1; kk < KS; ++kk) s = mfma32(kf[kk], qf[kk], s);
            __builtin_amdgcn_s_setprio(0);
            // next step's K fragments (the block's first after the last step)
            const int jn = j + 1 < nsub ? j + 1 : 0;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) kf[kk] = lds_k(jn, kk);
            if (!full && 32 * j + 32 > valid) {
                const int vj = valid - 32 * j;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (8 * (i >> 2) + 4 * hf + (i & 3) >= vj) s[i] = -INFINITY;
            }
            if (MASK) {
                const uint32_t bits = mrow[j];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (!((bits >> (8 * (i >> 2) + 4 * hf + (i & 3))) & 1u)) s[i] = -INFINITY;
            }
            // online softmax of the 32-key x 32-query tile
            float tm = fmaxf(s[0], s[1]);
#pragma unroll
            for (int i = 2; i < 16; ++i) tm = fmaxf(tm, s[i]);
            tm = halfwave_max(tm) * c;
            const bool up = tm > m + CK_TAU;
            const float mn = up ? tm : m;
            const float alpha = up ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
            m = mn;
            const float mref = MASK && mn == -INFINITY ? 0.0f : mn;
            uint32_t pw[8];
            float lsum = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // v_exp_f32 of arguments <= 8; results below 2^-126 flush to 0
                pw[k] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(s[2 * k], c, -mref)),
                                    __builtin_amdgcn_exp2f(fmaf(s[2 * k + 1], c, -mref)));
                lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[k]),
                                                       __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                                       lsum, false);
            }
            l = j == 0 ? lsum : l * alpha + lsum;
            const bf16x8 p0 = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
            const bf16x8 p1 = as_bf16x8(u32x4{pw[4], pw[5], pw[6], pw[7]});
            __builtin_amdgcn_s_setprio(1);
            if (j == 0) {
#pragma unroll
                for (int db = 0; db < 4; ++db) o[db] = mfma32(vf[db], p0, f32x16{});
            } else {
                if (__any(up)) {
#pragma unroll
                    for (int db = 0; db < 4; ++db)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
                }
#pragma unroll
                for (int db = 0; db < 4; ++db) o[db] = mfma32(vf[db], p0, o[db]);
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] = mfma32(vf[4 + db], p1, o[db]);
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int t = 0; t < 8; ++t) vf[t] = lds_v(jn, t);
        }
        store_partial(p, bh, chunk, q0, o, m, halfwave_sum(l), lane);
        if (!MASK) {
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) qf[kk] = qn[kk];
        }
    }
}

// MASK: the launch covers only the current-key chunks, attended under
// p.cur_mask (a separate instance, so that the mask's registers do not
// burden the history chunks' decode and attention).
template <int DK, bool MASK>
__global__ void __launch_bounds__(C8_THREADS, 1) chunk8_kernel(ChunkParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Chunk8Smem& sm = *reinterpret_cast<Chunk8Smem*>(smem_raw);
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    // history chunks first, (batch, head) fastest; then every current-key
    // chunk as cur_splits blocks over consecutive shares of the query blocks
    // (smaller work items where the grid drains)
    const int BH = p.B * p.H;
    const int64_t nh = (int64_t)p.nch_hist * BH;
    const int64_t item = (int64_t)blockIdx.x + p.blk_base;
    int bh, chunk, qb_lo = 0, qb_hi = p.qblocks;
    if (item < nh) {
        bh = (int)(item % BH);
        chunk = (int)(item / BH);
    } else {
        const int c = (int)(item - nh), ncur = p.nch_total - p.nch_hist;
        bh = c % BH;
        const int rest = c / BH;
        chunk = p.nch_hist + rest % ncur;
        const int qs = rest / ncur;
        qb_lo = (int)((int64_t)qs * p.qblocks / p.cur_splits);
        qb_hi = (int)((int64_t)(qs + 1) * p.qblocks / p.cur_splits);
    }
    const int b = bh / p.H, h = bh % p.H;
    const bool hist = chunk < p.nch_hist;
    const int64_t tok0 = (int64_t)(hist ? chunk : chunk - p.nch_hist) * CK_T;
    const int valid = (int)min((int64_t)CK_T, (hist ? p.n_rows : p.Nc) - tok0);

    if (!MASK && hist) fill_history8<DK>(sm, p, b, h, tok0, valid, t, wave, lane);
    else if (DK == CK_D) load_current_chunk8(sm, p, b, h, tok0, valid, t);
    __syncthreads();
    attend8<DK, MASK>(sm, p, b, h, bh, chunk, wave, lane, (valid + 31) / 32, valid, qb_lo, qb_hi,
                      tok0);
}

// ===================================================== staged schedule
// Stage: each 256-key chunk of (b, h) is decoded (history) or loaded
// (current keys) into LDS exactly as for the key-chunk kernel, then written
// to the workspace as two 128-key tiles.  A tile is two row-major images,
// the K rows [128 keys][128] and the V^T rows [128 d][128] (keys in V^T
// column order), unpadded: every 128-byte line of an image is written whole,
// and the flash kernel copies a tile into LDS with 1 KB direct-to-LDS loads
// whose sources place 16-byte chunk c of row r at chunk c ^ (r % 16), so that
// its operand reads of 16 consecutive rows hit distinct banks.
// Flash: one block of eight waves per (b*h, query tile, key split).  Wave w
// attends query block qt * qpt + w to the split's tiles, which stream
// through two LDS buffers, and keeps O, the running max and the row sum in
// registers across the whole split; the split's partial goes to the combine
// as a key-chunk partial (chunk index = split).  Next to the key-chunk
// schedule this trades the per-chunk partials of every query block (3x the
// decoded K/V) for one write and a few L2/MALL re-reads of the decoded K/V.
constexpr int FT_T = 128;                      // keys per tile
constexpr int FT_ROW = CK_D;                   // row pitch of both images (elements)
constexpr int FT_IMG = FT_T * FT_ROW;          // elements per V^T image (and K at DK = 128)
constexpr int FT_TILE = 2 * FT_IMG;            // K image, then V^T image (DK = 128)

// Tile geometry at K/Q width DK: the K image [128 keys][DK], then the V^T
// image [128 d][128].  K row r keeps logical 16-byte chunk c at chunk
// c ^ kswz(r), V^T row r at c ^ (r % 16), so that 16 consecutive rows read at
// one logical chunk hit distinct banks (rows of 16 chunks fill all 64 banks,
// rows of 8 or 4 chunks repeat every 2 or 4 rows).
template <int DK>
struct TileFmt {
    static constexpr int K_IMG = FT_T * DK;         // elements
    static constexpr int TILE = K_IMG + FT_IMG;     // elements
    static constexpr int CPR = DK / 8;              // chunks per K row
    static constexpr int K_PIECES = K_IMG * 2 / 1024;
    static constexpr int PIECES = TILE * 2 / 1024;
    __device__ static int kswz(int r) { return (r / (16 / CPR)) % CPR; }
};
static_assert(TileFmt<32>::K_IMG * 2 % 1024 == 0, "a K image must be whole 1 KB pieces");
static_assert(TileFmt<32>::TILE == FT_T * 32 + FT_IMG && TileFmt<64>::TILE == FT_T * 64 + FT_IMG &&
                  TileFmt<CK_D>::TILE == FT_TILE,
              "the tile format and the workspace plan must agree on a tile's size");

// Elements of one tile image pair (K, then V^T) and of its K image at K/Q
// width dk, from the same TileFmt the kernels address the tiles with.
size_t tile_elems(int dk) {
    return dk == 32 ? TileFmt<32>::TILE : dk == 64 ? TileFmt<64>::TILE : TileFmt<CK_D>::TILE;
}
size_t k_image_elems(int dk) {
    return dk == 32 ? TileFmt<32>::K_IMG : dk == 64 ? TileFmt<64>::K_IMG : TileFmt<CK_D>::K_IMG;
}
static_assert(CK_T == 2 * FT_T, "two tiles per chunk");

// s_waitcnt vmcnt(0) lgkmcnt(0): the wave's loads have landed and its LDS
// reads are done
__device__ __forceinline__ void wait_loads_and_lds() { __builtin_amdgcn_s_waitcnt(7 << 4); }

__global__ void __launch_bounds__(C8_THREADS, 1) stage8_kernel(ChunkParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Chunk8Smem& sm = *reinterpret_cast<Chunk8Smem*>(smem_raw);
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int BH = p.B * p.H;
    const int bh = (int)(blockIdx.x % BH), chunk = (int)(blockIdx.x / BH);
    const int b = bh / p.H, h = bh % p.H;
    const int nch_hist = p.ntiles_hist / 2;
    const bool hist = chunk < nch_hist;
    const int64_t tok0 = (int64_t)(hist ? chunk : chunk - nch_hist) * CK_T;
    const int valid = (int)min((int64_t)CK_T, (hist ? p.n_rows : p.Nc) - tok0);
    if (hist) fill_history8<CK_D>(sm, p, b, h, tok0, valid, t, wave, lane);
    else load_current_chunk8(sm, p, b, h, tok0, valid, t);
    __syncthreads();
    uint16_t* dst = p.tiles + ((int64_t)bh * p.ntiles + 2 * chunk) * FT_TILE;
    // a second half with no valid key is never attended: not written
    const int halves = valid > FT_T ? 2 : 1;
    for (int hh = 0; hh < halves; ++hh) {
        u32x4* kd = reinterpret_cast<u32x4*>(dst + hh * FT_TILE);
        u32x4* vd = reinterpret_cast<u32x4*>(dst + hh * FT_TILE + FT_IMG);
        // K rows 128 hh .. +128 without their LDS padding
        for (int i = t; i < FT_T * (FT_ROW / 8); i += C8_THREADS)
            kd[i] = *reinterpret_cast<const u32x4*>(&sm.k[FT_T * hh + (i >> 4)][8 * (i & 15)]);
        // V^T: the 16 pieces of keys 128 hh .. +128 of each d row
        for (int i = t; i < CK_D * 16; i += C8_THREADS) {
            const int d = i >> 4, c = i & 15;
            vd[d * (FT_ROW / 8) + c] = *reinterpret_cast<const u32x4*>(&sm.vt[d][FT_T * hh + 8 * c]);
        }
    }
}

// ------------------------------------------------------------ current tiles
// Current-key tiles (the uncompressed keys of the chunk being attended) are
// built by the current-key blocks of drtile_kernel (ctile_batch).

// ------------------------------------------------ decode GEMM, resident decoder
// For codec ranks up to DR_MAXQ * 64 the history tiles come from drtile_kernel:
// a block of eight waves decoding a piece of one head's tiles (a range of
// tiles, see drtile_pieces) loads the head's decoder rows into LDS once and
// keeps them for the whole piece, so each decoder element is read from L2
// once per piece rather than once per 256-key chunk.  The block decodes two
// tiles at a time: wave w takes keys
// 32 (w % 4) .. +32 of tile 2 i + w / 4 at all 128 columns, so each unpacked
// INT4 code feeds four MFMAs, and stores its part of the image from
// registers (each 128-byte line of a K row is written by one wave, each line
// of a V^T row by two).  The center rows of every key of the range are
// resolved once, into LDS, before the first tile, so the tile loop writes no
// LDS and needs no barrier: each wave runs its tiles at its own pace, one
// wave's epilogue overlapping another's GEMM on the same SIMD.  Codes are
// fetched one pair of tiles ahead; the center values of a pair are requested
// before its GEMM and used after it.
constexpr int DR_THREADS = 512;
constexpr int DR_MAXQ = 6;             // 64-rank decoder slices held: r <= 384
constexpr int DR_SLICE = CK_D * 64;    // elements per slice
constexpr int DR_MAXT = 24;            // tiles per block (the center-row table)
constexpr int DR_SROW = 40;            // staging row: 32 values + 8 of padding (80 B)
struct DResSmem {
    uint16_t dec[DR_MAXQ * DR_SLICE];      // slice s at s * DR_SLICE: [128 rows][64], chunks swizzled
    const uint16_t* crow[DR_MAXT * FT_T];  // center row of key k of tile ta + k / 128
    float bias[CK_D];
    uint16_t stage[DR_THREADS / 64][32 * DR_SROW];  // per wave: one 32 x 32 slice of its output
};
static_assert(sizeof(DResSmem) <= 160 * 1024, "LDS budget");

// A key's center row as a reference loaded ahead of its use: the row is
// base + clamp(id, 0, nc - 1) * c_rs (the id is the only value that waits on
// memory when the reference is formed).
struct CenterRef {
    const uint16_t* base;
    int id, nc;
};

__device__ __forceinline__ CenterRef center_ref(const ChunkCodec& c, int b, int h, int64_t N,
                                                int64_t row) {
    if (c.seg) {
        const NKV_GLOBAL nkv_segment& s = seg_at(c.seg, seg_find(c.seg, c.n_seg, row));
        const int64_t local = min(max(row - s.row_start, (int64_t)0), s.rows - 1);
        const uint16_t* base =
            c.seg_flat ? c.centers + (int64_t)b * c.c_bs + s.center_base * c.c_rs + (int64_t)h * c.c_hs
                       : s.centers + (int64_t)b * s.centers_batch_stride + (int64_t)h * c.c_hs;
        return {base, read_id(s.ids, s.id_bytes, (int64_t)b * s.rows + local), s.num_centers};
    }
    return {c.centers + (int64_t)b * c.c_bs + (int64_t)h * c.c_hs,
            read_id(c.ids, c.id_bytes, (int64_t)b * N + row), c.num_centers};
}

__device__ __forceinline__ const uint16_t* center_ptr(const CenterRef& r, int64_t c_rs) {
    return r.base + (int64_t)min(max(r.id, 0), r.nc - 1) * c_rs;
}

// One codec of tiles [ta, tb) (tb - ta <= DR_MAXT) of head bh, two at a time
// (pair i: tiles ta + 2 i and ta + 2 i + 1), K at width DK (V at 128).
template <int CODEC, int KQ, int DK>
__device__ __forceinline__ void drtile_range(DResSmem& sm, const ChunkParams& p, int bh, int ta,
                                             int tb, int wave, int lane) {
    using TF = TileFmt<DK>;
    constexpr int W = CODEC == 0 ? DK : CK_D;  // decoded columns
    constexpr int NDT = W / 32;                 // 32-column MFMA tiles per wave
    const ChunkCodec& cd = p.codec[CODEC];
    const int t = threadIdx.x, hf = lane >> 5, l32 = lane & 31;
    const int kq = wave & 3, tp = wave >> 2;
    const int b = bh / p.H, h = bh % p.H;
    // head of the center table and bias
    const int hc = cd.c_heads ? min(max(ldg(cd.c_heads + h), 0), cd.c_heads_n - 1) : h;
    const int R = cd.r, G = cd.group;
    const bool cent = cd.has_centers, f16 = cd.scale_dtype == NKV_DTYPE_FP16;
    // the head's decoder rows, KQ slices of W / 8 pieces (8 rows x 128 B)
    // taken by the waves in turn: lane L of a piece brings logical chunk
    // (L % 8) ^ ((row >> 1) & 7) of its row 8 piece + L / 8
    {
        const uint16_t* wsrc = cd.w + (int64_t)h * cd.w_hs;
        for (int e = wave; e < KQ * (W / 8); e += DR_THREADS / 64) {
            const int s = e / (W / 8), pc = e % (W / 8), row = 8 * pc + (lane >> 3);
            const int ch = (lane & 7) ^ ((row >> 1) & 7);
            __builtin_amdgcn_global_load_lds(wsrc + (int64_t)row * R + 64 * s + 8 * ch,
                                             NKV_LDS(sm.dec + s * DR_SLICE + pc * 512), 16, 0, 0);
        }
    }
    if (t < W) sm.bias[t] = cd.bias ? bf16_round(cd.bias[(int64_t)hc * cd.bias_hs + t]) : 0.0f;
    // codec row of key k of tile `tile`; keys past the last row take key 0's
    // codes and center (finite, never attended)
    auto key_row = [&](int tile, int k) {
        const int64_t tok0 = (int64_t)tile * FT_T;
        const int valid = (int)min((int64_t)FT_T, p.n_rows - tok0);
        return history_row(p, tok0 + (k < valid ? k : 0));
    };
    // this lane's key: 32 kq + l32 of tile 2 i + tp of the pair
    const int key = 32 * kq + l32;
    // scale of this lane's ranks 64 s + 32 hf .. +32 (one group: group % 32 == 0)
    int sidx[KQ];
#pragma unroll
    for (int s = 0; s < KQ; ++s) sidx[s] = (64 * s + 32 * hf) / G;
    auto fetch = [&](int tile, u32x4 (&pk)[KQ], uint16_t (&sc)[KQ]) {
        const uint8_t* prow;
        const uint16_t* srow;
        codec_row_ptrs(cd, b, p.N, key_row(tile < tb ? tile : ta, key), prow, srow);
        prow += 16 * hf;
#pragma unroll
        for (int s = 0; s < KQ; ++s) {
            pk[s] = ldg(reinterpret_cast<const u32x4*>(prow + 32 * s));
            sc[s] = ldg(srow + sidx[s]);
        }
    };
    // center values of this lane's tile (table rows from crow): K, the
    // columns 32 dt + 8 g + 4 hf .. +4 of this lane's key; V, column
    // d = 32 dt + l32 of keys 32 kq + 8 g + 4 hf + e
    constexpr int NCV = CODEC == 0 ? 8 * NDT : 64;
    // K: row (lane >> 2) + 16 i of the wave's 32 keys at columns 32 dt +
    // 8 (lane & 3) .. +8 (added when the staged rows are flushed), so that
    // each load reads 16 rows x 64 contiguous bytes rather than 32 rows x 16
    // bytes.
    auto load_centers = [&](uint32_t (&cv)[NCV], const uint16_t* const* crow) {
        if (CODEC == 0) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint16_t* cr = crow[32 * kq + (lane >> 2) + 16 * i];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x4 v = ldg(reinterpret_cast<const u32x4*>(cr + 32 * dt + 8 * (lane & 3)));
#pragma unroll
                    for (int w = 0; w < 4; ++w) cv[4 * (2 * dt + i) + w] = v[w];
                }
            }
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t* cr = crow[32 * kq + 8 * g + 4 * hf + e];
#pragma unroll
                    for (int dt = 0; dt < 4; ++dt) cv[16 * dt + 4 * g + e] = ldg(cr + 32 * dt + l32);
                }
        }
    };
    int wofs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wofs[j] = l32 * 64 + 8 * ((4 * hf + j) ^ ((l32 >> 1) & 7));
    u32x4 pk[KQ], pn[KQ];
    uint16_t sc[KQ], sn[KQ];
    uint32_t cv[NCV];
    fetch(ta + tp, pk, sc);
    // the center row of every key of the range: all references are requested
    // before the first is resolved
    if (cent) {
        constexpr int PER = DR_MAXT * FT_T / DR_THREADS;
        const int nk = (tb - ta) * FT_T;
        CenterRef r[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int k = t + e * DR_THREADS;
            if (k < nk) r[e] = center_ref(cd, b, hc, p.N, key_row(ta + (k >> 7), k & 127));
        }
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int k = t + e * DR_THREADS;
            if (k < nk) sm.crow[k] = center_ptr(r[e], cd.c_rs);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    const int npairs = (tb - ta + 1) / 2;
    for (int i = 0; i < npairs; ++i) {
        const int tile = ta + 2 * i + tp;
        // the last pair of an odd range has no second tile: its waves are done
        if (tile >= tb) break;
        if (cent) load_centers(cv, sm.crow + (tile - ta) * FT_T);
        if (tile + 2 < tb) fetch(tile + 2, pn, sn);
        f32x16 acc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x16{};
#pragma unroll
        for (int s = 0; s < KQ; ++s) {
            const float scl = f16 ? f16_bits_to_f32(sc[s]) : bf16_bits_to_f32(sc[s]);
            const float ns7 = -7.0f * scl;
            const uint16_t* ws = sm.dec + s * DR_SLICE;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x8 z = unpack8(pk[s][j], scl, ns7);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const bf16x8 w = lds_b128(ws + 32 * dt * 64 + wofs[j]);
                    acc[dt] = CODEC == 0 ? mfma32(w, z, acc[dt]) : mfma32(z, w, acc[dt]);
                }
            }
        }
        {
            uint16_t* img = p.tiles + ((int64_t)bh * p.ntiles + tile) * TF::TILE + CODEC * TF::K_IMG;
            // Each 32-column slice dt of the wave's output goes through its own
            // LDS staging rows, then out as 64 contiguous bytes per row (four
            // lanes of 16 B): K rows are the wave's 32 keys at columns 32 dt ..,
            // V^T rows 32 dt .. at the wave's 32 key columns.  Scattered 8-byte
            // stores from the accumulator layout would cost the L2 four times
            // the write requests.
            uint16_t* st = sm.stage[wave];
            auto flush = [&](int dt) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int r = (lane >> 2) + 16 * i, c = lane & 3;
                    const u32x4 x = *reinterpret_cast<const u32x4*>(st + r * DR_SROW + 8 * c);
                    uint16_t* dst = CODEC == 0 ? img + (32 * kq + r) * DK + 32 * dt + 8 * c
                                               : img + (32 * dt + r) * FT_ROW + 32 * kq + 8 * c;
                    if (CODEC == 0 && cent) {
                        // K = bf16(bf16(acc + bias) + center) (MG:438-454)
                        u32x4 y;
#pragma unroll
                        for (int w = 0; w < 4; ++w) {
                            const uint32_t cw = cv[4 * (2 * dt + i) + w];
                            y[w] = pack_bf16x2(__uint_as_float(x[w] << 16) + __uint_as_float(cw << 16),
                                               __uint_as_float(x[w] & 0xffff0000u) +
                                                   __uint_as_float(cw & 0xffff0000u));
                        }
                        *reinterpret_cast<u32x4*>(dst) = y;
                    } else {
                        *reinterpret_cast<u32x4*>(dst) = x;
                    }
                }
            };
            if (CODEC == 0) {
                // acc[dt] element i: d = 32 dt + 8 (i/4) + 4 hf + i%4 of this
                // lane's key; K = bf16(bf16(acc + bias) + center), the center
                // added in flush() from coalesced rows (read-time RoPE and the
                // camera follow in tile_xform_kernel)
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int d = 32 * dt + 8 * g + 4 * hf;
                        const f32x4 bs = *reinterpret_cast<const f32x4*>(&sm.bias[d]);
                        float a[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) a[e] = acc[dt][4 * g + e] + bs[e];
                        *reinterpret_cast<u32x2*>(st + l32 * DR_SROW + 8 * g + 4 * hf) =
                            u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
                    }
                    flush(dt);
                }
            } else {
                // acc[dt] element i: key 32 kq + 8 (i/4) + 4 hf + i%4, d = 32 dt
                // + l32; V = bf16(bf16(acc + bias) + center), written to V^T in
                // the attention's column order
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const float bs = sm.bias[32 * dt + l32];
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        float v[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float a = bf16_round(acc[dt][4 * g + e] + bs);
                            v[e] = cent ? a + __uint_as_float((cv[16 * dt + 4 * g + e] & 0xffffu) << 16) : a;
                        }
                        *reinterpret_cast<u32x2*>(st + l32 * DR_SROW + vt_col(8 * g + 4 * hf)) =
                            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    }
                    flush(dt);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < KQ; ++s) {
            pk[s] = pn[s];
            sc[s] = sn[s];
        }
    }
}

// Entry i of a camera's fp64 matrix table (the tile pass reads it): entry e
// of set s is bf16(mats[batch][m][e]), s = batch * n_mats + m.
__device__ __forceinline__ void camera_table_entry(const CameraDev& c, int batches, int64_t i) {
    const int64_t per = (int64_t)c.n_mats * 64;
    if (i >= batches * per) return;
    const int64_t b = i / per, r = i - b * per;
    const_cast<double*>(c.m64)[i] = (double)bf16_round(ldg(c.mats + b * c.mats_bs + r));
}

// Range j of nb equal ranges of the partition's B*H*T history tiles
// (head-major), one head piece of at most DR_MAXT tiles at a time.
template <int CODEC, int KQ, int DK>
__device__ __forceinline__ void drtile_pieces(DResSmem& sm, const ChunkParams& p, int64_t j, int nb,
                                              int wave, int lane) {
    const int T = (int)cdiv(p.n_rows, FT_T);
    const int64_t M = (int64_t)p.B * p.H * T, start = j * M / nb, end = (j + 1) * M / nb;
    for (int64_t pos = start; pos < end;) {
        const int hb = (int)(pos / T), ta = (int)(pos - (int64_t)hb * T);
        const int tb = (int)min((int64_t)min(T, ta + DR_MAXT), ta + (end - pos));
        if (pos > start) __syncthreads();  // the previous piece's LDS reads are done
        drtile_range<CODEC, KQ, DK>(sm, p, hb, ta, tb, wave, lane);
        pos += tb - ta;
    }
}

// Current tiles x0, x0 + stride, .. (up to CJ_BATCH of them below `jobs`;
// tile x is current tile x % nct of head x / nct) by the DR_THREADS threads
// of a current-key block, every K and V load of the batch issued before the
// first store, each load instruction reading four whole 256-byte rows: K
// rows straight into the image (16-byte piece t + DR_THREADS e of a tile is
// column block piece % 16 of key piece / 16), V through LDS into V^T column
// order (thread t: columns 8 (t % 16) .. +8 of keys 4 (t / 16) .. +4, one
// 8-byte write of four keys per column).  The LDS V^T rows hold their
// 16-byte chunk c at chunk c ^ ((row / 8) % 16), so that the 16 rows one
// such write instruction touches per key group fall in distinct banks.
// Keys past the end are zero.
constexpr int CJ_PIECES = FT_T * CK_D / 8 / DR_THREADS;  // 16-byte pieces per thread and tile
constexpr int CJ_BATCH = 4;
static_assert(CJ_PIECES == 4 && DR_THREADS == 512, "current tile batches");
static_assert(CJ_BATCH * FT_IMG * sizeof(uint16_t) <= sizeof(DResSmem), "V^T images in the decode LDS");

__device__ __forceinline__ void ctile_batch(const ChunkParams& p, int x0, int stride, int jobs,
                                            int nct, uint16_t* vt, int t) {
    const int k0 = 4 * (t >> 4), d0 = 8 * (t & 15);
    u32x4 kv[CJ_BATCH][CJ_PIECES], vv[CJ_BATCH][4];
    int64_t img0[CJ_BATCH];  // element offset of each tile's image (32-bit division only)
#pragma unroll
    for (int m = 0; m < CJ_BATCH; ++m) {
        const int x = x0 + m * stride, bh = x / nct, ct = x - bh * nct;
        const int b = bh / p.H, h = bh - b * p.H;
        img0[m] = ((int64_t)bh * p.ntiles + p.ntiles_hist + ct) * FT_TILE;
        const int64_t key0 = (int64_t)ct * FT_T;
        const int valid = x < jobs ? (int)min((int64_t)FT_T, p.Nc - key0) : 0;
        const uint16_t* ks = p.k_cur + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
        const uint16_t* vs = p.v_cur + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + d0;
#pragma unroll
        for (int e = 0; e < CJ_PIECES; ++e) {
            const int i = t + DR_THREADS * e, key = i >> 4, c = i & 15;
            kv[m][e] = key < valid ? ldg(reinterpret_cast<const u32x4*>(ks + (key0 + key) * p.k_st + 8 * c))
                                   : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
            vv[m][e] = k0 + e < valid ? ldg(reinterpret_cast<const u32x4*>(vs + (key0 + k0 + e) * p.v_st))
                                      : u32x4{0, 0, 0, 0};
    }
    // V^T column of key k0 (its four keys are adjacent there), then its
    // 16-byte chunk swizzled per row group
    const int col = vt_col(k0), vch = col >> 3, vin = col & 7;
#pragma unroll
    for (int m = 0; m < CJ_BATCH; ++m) {
        if (x0 + m * stride < jobs) {
            uint16_t* img = p.tiles + img0[m];
#pragma unroll
            for (int e = 0; e < CJ_PIECES; ++e) {
                const int i = t + DR_THREADS * e;
                *reinterpret_cast<u32x4*>(img + (i >> 4) * FT_ROW + 8 * (i & 15)) = kv[m][e];
            }
        }
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
            const int w = dd >> 1, sh = 16 * (dd & 1);
            auto val = [&](int e) { return (vv[m][e][w] >> sh) & 0xffffu; };
            const int row = d0 + dd;
            *reinterpret_cast<u32x2*>(vt + m * FT_IMG + row * FT_ROW + 8 * (vch ^ ((row >> 3) & 15)) + vin) =
                u32x2{val(0) | (val(1) << 16), val(2) | (val(3) << 16)};
        }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < CJ_BATCH; ++m) {
        if (x0 + m * stride >= jobs) break;
        uint16_t* img = p.tiles + img0[m] + FT_IMG;
#pragma unroll
        for (int e = 0; e < CJ_PIECES; ++e) {
            const int i = t + DR_THREADS * e, row = i >> 4, c = i & 15;
            *reinterpret_cast<u32x4*>(img + 8 * i) = *reinterpret_cast<const u32x4*>(
                vt + m * FT_IMG + row * FT_ROW + 8 * (c ^ ((row >> 3) & 15)));
        }
    }
    __syncthreads();  // the LDS images are read before the next batch rewrites them
}

// Blocks of a decode segment: seg_ranges equal ranges of the segment's
// history tiles (see the kernel body).  Blocks of a current-key segment:
// seg_ranges blocks, block c building the partition's current tiles c,
// c + seg_ranges, .. in batches.  KQ: decoder slices of the launch's decode
// segments.
template <int KQ>
__global__ void __launch_bounds__(DR_THREADS, 1) drtile_kernel(MultiParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sg = multi_segment(P, blockIdx.x);
    const int pi = P.seg_part[sg], kind = P.seg_kind[sg], dk = P.dk[pi];
    const ChunkParams& p = P.part[pi];
    const int64_t local = (int64_t)blockIdx.x - P.seg_first[sg];
    const int BH = p.B * p.H;
    if (kind == SEG_TABLE) {
        camera_table_entry(p.cam, camera_batches(p.cam, p.B), local * DR_THREADS + threadIdx.x);
        return;
    }
    if (kind == SEG_CUR) {
        // (B*H*nct < 2^31: checked on the host)
        const int ncur = P.seg_ranges[sg], nct = p.ntiles - p.ntiles_hist, jobs = BH * nct;
        for (int x0 = (int)local; x0 < jobs; x0 += CJ_BATCH * ncur)
            ctile_batch(p, x0, ncur, jobs, nct, reinterpret_cast<uint16_t*>(smem_raw), threadIdx.x);
        return;
    }
    // a decode segment of nb blocks (a multiple of 8): range j of the
    // segment's B*H*T history tiles, head-major -- ranges j .. of one XCD
    // adjacent, so that they share decoder rows in its L2 -- one head piece
    // at a time
    DResSmem& sm = *reinterpret_cast<DResSmem*>(smem_raw);
    const int nb = P.seg_ranges[sg];
    const int64_t j = nb % 8 == 0 ? (local & 7) * (nb >> 3) + (local >> 3) : local;
    if (kind == SEG_K) {
        if (dk == 32) drtile_pieces<0, KQ, 32>(sm, p, j, nb, wave, lane);
        else if (dk == 64) drtile_pieces<0, KQ, 64>(sm, p, j, nb, wave, lane);
        else drtile_pieces<0, KQ, 128>(sm, p, j, nb, wave, lane);
    } else {
        if (dk == 32) drtile_pieces<1, KQ, 32>(sm, p, j, nb, wave, lane);
        else if (dk == 64) drtile_pieces<1, KQ, 64>(sm, p, j, nb, wave, lane);
        else drtile_pieces<1, KQ, 128>(sm, p, j, nb, wave, lane);
    }
}

// ---------------------------------------- read-time transforms of the tiles
// Read-time RoPE and the camera's FULL layout are applied to the decode
// GEMM's history tiles in place, after the decode launch and before the flash
// launch (drtile_kernel's epilogue has no registers to spare for them): one
// block of TX_THREADS threads per history tile.  The block first issues its
// first tile loads, then resolves each key's tables once into LDS (its RoPE
// band rows and its camera matrix set), then transforms the tile in groups
// of TX_GROUP words per thread.  K: each 32-bit word is one pair of a key
// row; RoPE rotates pair pp (or, for a reader key, its original pair
// rope.pairs[h][pp], rope_selected CN/core.py:75-91) at the key's codec row
// (rope_k_rows' arithmetic).  The camera multiplies the two 4-vectors of
// each 8-dim block j of a key -- the block's even and odd dims, i.e. the low
// and high halves of its four pair words, which sit in one quad of lanes --
// by sub-frame j % 4 of P^-1 (a 128-wide key and every value: the FULL
// layout, prope_attention.py:120-176) or cam.blocks[h][j] (a reader key,
// camera_selected CN/core.py:110-137); lane w of the quad computes output w
// of both.  V^T: a lane holds two key columns of the 8 rows of block j.
// This is the arithmetic of the key-chunk kernel's camera passes
// (camera_k_rows and the V^T pass of decode_codec8) on the same bf16
// values, so both schedules write bit-identical K and V.
constexpr int TX_THREADS = 256;
constexpr int TX_GROUP = 8;  // K words of a thread in flight at once
struct TXformSmem {
    const double* band[3][FT_T];  // RoPE: the t, h and w band rows of each key's codec row
    const double* mats[FT_T];     // camera: each key's sub-frame matrices in the fp64 table
};

// m_row . x for one row of a matrix of the fp64 table (entries rounded to
// bf16) and a 4-vector x of bf16 values: camera_vec4's sum, in order, in
// fp64.  Every product of two bf16 values is exact in fp64, so a fused
// multiply-add rounds exactly as the sum of the product does.
__device__ __forceinline__ float camera_dot64(const double* m_row, const float (&x)[4]) {
    const f64x2 a = ldg(reinterpret_cast<const f64x2*>(m_row));
    const f64x2 c = ldg(reinterpret_cast<const f64x2*>(m_row) + 1);
    double acc = a.x * (double)x[0];
    acc = __builtin_fma(a.y, (double)x[1], acc);
    acc = __builtin_fma(c.x, (double)x[2], acc);
    acc = __builtin_fma(c.y, (double)x[3], acc);
    return bf16_round(f64_to_f32(acc));
}

// Lane q of every quad (lanes 4 a .. 4 a + 4) receives v of lane 4 a + Q.
template <int Q>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, Q * 0x55, 0xf, 0xf, false);
}

template <int DK>
__device__ __forceinline__ void tile_xform(TXformSmem& sm, const ChunkParams& p, int bh, int tile,
                                           int t) {
    using TF = TileFmt<DK>;
    constexpr int PPR = DK / 2;            // pair words per K row
    constexpr int RPI = TX_THREADS / PPR;  // K rows per pass of the block
    constexpr int KU = FT_T / RPI;         // K words per thread
    static_assert(KU % TX_GROUP == 0, "whole groups of K words");
    const int b = bh / p.H, h = bh % p.H;
    const int64_t tok0 = (int64_t)tile * FT_T;
    const int valid = (int)min((int64_t)FT_T, p.n_rows - tok0);
    const bool rope = rope_on(p.rope), cam = p.cam.mats != nullptr;
    // a reader key without a block map keeps its values under the camera,
    // as in camera_k_rows
    const int32_t* blocks = p.cam.blocks ? p.cam.blocks + (int64_t)h * (DK / 8) : nullptr;
    const bool kcam = cam && (blocks || DK == CK_D);
    uint16_t* img = p.tiles + ((int64_t)bh * p.ntiles + tile) * TF::TILE;
    // K: thread t takes pair pp of key rows t / PPR + RPI i (a wave reads
    // whole rows); keys past the last row keep their K
    const int pp = t % PPR, r0 = t / PPR;
    uint32_t* kw = reinterpret_cast<uint32_t*>(img) + pp;
    auto load_group = [&](int g, uint32_t (&kx)[TX_GROUP]) {
#pragma unroll
        for (int i = 0; i < TX_GROUP; ++i) {
            const int k = r0 + RPI * (g + i);
            kx[i] = k < valid ? kw[k * PPR] : 0u;
        }
    };
    uint32_t kx[TX_GROUP];
    if (rope || kcam) load_group(0, kx);
    // V^T: wave v takes blocks j = 4 v .. 4 v + 4 (sub-frames 0 .. 3), rows
    // 8 j .. 8 j + 8 at key columns 2 lane, 2 lane + 1, each block's rows
    // loaded one block ahead (the first with K's); the finite columns of
    // keys past the last row are never attended
    const int lane = t & 63, v = t >> 6;
    uint32_t* vw = reinterpret_cast<uint32_t*>(img + TF::K_IMG) + lane;
    auto load_v = [&](int jj, uint32_t (&vx)[8]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vx[e] = vw[(8 * (4 * v + jj) + e) * (FT_ROW / 2)];
    };
    uint32_t vx[8];
    if (cam) load_v(0, vx);
    // each key's tables, once (keys past the last row take key 0's)
    if (t < FT_T) {
        const int64_t row = history_row(p, tok0 + (t < valid ? t : 0));
        if (rope) {
            const RopeRows rr = rope_rows(p.rope, row);
            sm.band[0][t] = rr.t;
            sm.band[1][t] = rr.h;
            sm.band[2][t] = rr.w;
        }
        if (cam) sm.mats[t] = p.cam.m64 + 64 * camera_set(p.cam, b, row);
    }
    __syncthreads();
    if (rope || kcam) {
        // this lane's pair: its RoPE band and entry, its block and sub-frame
        int band = 0, off = 0;
        if (rope) {
            int pj = p.rope.pairs ? ldg(p.rope.pairs + (int64_t)h * PPR + pp) : pp;
            pj = min(max(pj, 0), p.rope.pt + p.rope.ph + p.rope.pw - 1);
            band = pj < p.rope.pt ? 0 : (pj < p.rope.pt + p.rope.ph ? 1 : 2);
            off = 2 * (pj - (band == 0 ? 0 : band == 1 ? p.rope.pt : p.rope.pt + p.rope.ph));
        }
        const int j = pp >> 2, w = pp & 3;
        const int sub = kcam ? (blocks ? ldg(blocks + j) & 3 : j & 3) : 0;
        for (int g = 0; g < KU; g += TX_GROUP) {
            if (g > 0) load_group(g, kx);
            if (rope) {
                // global loads (generic pointers from LDS would make flat
                // loads, which wait with the LDS reads)
                f64x2 cs[TX_GROUP];
#pragma unroll
                for (int i = 0; i < TX_GROUP; ++i) {
                    const int k = min(r0 + RPI * (g + i), valid - 1);
                    cs[i] = ldg(reinterpret_cast<const f64x2*>(sm.band[band][k] + off));
                }
#pragma unroll
                for (int i = 0; i < TX_GROUP; ++i) kx[i] = rope_pair(kx[i], cs[i].x, cs[i].y);
            }
            if (kcam) {
#pragma unroll
                for (int i = 0; i < TX_GROUP; ++i) {
                    const int k = min(r0 + RPI * (g + i), valid - 1);
                    const uint32_t q0 = quad_bcast<0>(kx[i]), q1 = quad_bcast<1>(kx[i]);
                    const uint32_t q2 = quad_bcast<2>(kx[i]), q3 = quad_bcast<3>(kx[i]);
                    const float x0[4] = {__uint_as_float(q0 << 16), __uint_as_float(q1 << 16),
                                         __uint_as_float(q2 << 16), __uint_as_float(q3 << 16)};
                    const float x1[4] = {__uint_as_float(q0 & 0xffff0000u),
                                         __uint_as_float(q1 & 0xffff0000u),
                                         __uint_as_float(q2 & 0xffff0000u),
                                         __uint_as_float(q3 & 0xffff0000u)};
                    const double* mr = sm.mats[k] + 16 * sub + 4 * w;
                    kx[i] = pack_bf16x2(camera_dot64(mr, x0), camera_dot64(mr, x1));
                }
            }
#pragma unroll
            for (int i = 0; i < TX_GROUP; ++i) {
                const int k = r0 + RPI * (g + i);
                if (k < valid) kw[k * PPR] = kx[i];
            }
        }
    }
    if (cam) {
        const double* mk[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) mk[c] = sm.mats[vt_col(2 * lane + c)];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int j = 4 * v + jj;
            uint32_t vn[8];
            if (jj < 3) load_v(jj + 1, vn);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int sh = 16 * c;
                float x0[4], x1[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x0[i] = __uint_as_float(((vx[2 * i] >> sh) & 0xffffu) << 16);
                    x1[i] = __uint_as_float(((vx[2 * i + 1] >> sh) & 0xffffu) << 16);
                }
                const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const double* mrow = mk[c] + 16 * jj + 4 * i;
                    const float y0 = camera_dot64(mrow, x0), y1 = camera_dot64(mrow, x1);
                    vx[2 * i] = (vx[2 * i] & keep) | ((uint32_t)f32_to_bf16_bits(y0) << sh);
                    vx[2 * i + 1] = (vx[2 * i + 1] & keep) | ((uint32_t)f32_to_bf16_bits(y1) << sh);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) vw[(8 * j + e) * (FT_ROW / 2)] = vx[e];
            if (jj < 3) {
#pragma unroll
                for (int e = 0; e < 8; ++e) vx[e] = vn[e];
            }
        }
    }
}

// Blocks of a transform segment: the partition's history tiles, tile
// fastest within each b*h.
__global__ void __launch_bounds__(TX_THREADS) tile_xform_kernel(MultiParams P) {
    __shared__ TXformSmem sm;
    const int sg = multi_segment(P, blockIdx.x);
    const int pi = P.seg_part[sg];
    const ChunkParams& p = P.part[pi];
    const int64_t local = (int64_t)blockIdx.x - P.seg_first[sg];
    const int T = (int)cdiv(p.n_rows, FT_T);
    const int bh = (int)(local / T), tile = (int)(local % T);
    if (P.dk[pi] == 32) tile_xform<32>(sm, p, bh, tile, threadIdx.x);
    else if (P.dk[pi] == 64) tile_xform<64>(sm, p, bh, tile, threadIdx.x);
    else tile_xform<CK_D>(sm, p, bh, tile, threadIdx.x);
}

// The two tile buffers as [K0][K1][V0][V1]: a buffer's images sit one
// image from the other buffer's, so that every operand read is one per-lane
// register plus an immediate offset (below 64 KB) for both buffers.
template <int DK>
struct FlashSmem {
    uint16_t k[2][TileFmt<DK>::K_IMG];
    uint16_t v[2][FT_IMG];
};
static_assert(sizeof(FlashSmem<CK_D>) <= 160 * 1024, "LDS budget");
constexpr int FT_IMG_BYTES = FT_IMG * 2;

// Block blk of one partition at K/Q width DK.  MASK: the current keys are
// attended under p.cur_mask (the history tiles never are).
template <int DK, bool MASK>
__device__ __forceinline__ void flash_block(const ChunkParams& p, int64_t blk, unsigned char* smem_raw) {
    using TF = TileFmt<DK>;
    constexpr int K_BYTES = TF::K_IMG * 2;
    FlashSmem<DK>& sm = *reinterpret_cast<FlashSmem<DK>*>(smem_raw);
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Work items in group-major order (group g = (head, split) = bh + B*H *
    // split, then its qtiles query tiles), cut into eight equal runs, one
    // per XCD: block blk is dispatch slot blk / 8 of XCD blk % 8 (the
    // segment starts at a multiple of 8) and takes item (blk % 8) * per +
    // blk / 8.  The query tiles of a group then run on one XCD in
    // consecutive slots, streaming the same tiles at the same time, so that
    // XCD's L2 serves all but the first read of each tile; every XCD gets the
    // same number of items, the last run ending in empty blocks.
    const int BH = p.B * p.H;
    const int64_t items = (int64_t)BH * p.splits * p.qtiles, per = (items + 7) >> 3;
    const int64_t item = (blk & 7) * per + (blk >> 3);
    if (item >= items) return;
    const int g = (int)(item / p.qtiles), qt = (int)(item % p.qtiles);
    const int bh = g % BH, split = g / BH;
    const int b = bh / p.H, h = bh % p.H;
    const int t0 = (int)((int64_t)split * p.ntiles / p.splits);
    const int t1 = (int)((int64_t)(split + 1) * p.ntiles / p.splits);
    const int qb = qt * p.qpt + wave;
    const bool active = wave < p.qpt && qb < p.qblocks;
    // tile i of the split goes to buffer i % 2; piece e (1 KB) of a tile:
    // lane L brings chunk (L % CPR) ^ kswz(row) of K row 512 e / DK + L / CPR,
    // or chunk (L % 16) ^ (row % 16) of V^T row 4 e' + L / 16 (e' = e minus
    // the K pieces).  This wave's pieces are e = wave + 8 i: K_PIECES is a
    // multiple of 8 and both swizzles repeat every 16 rows (4 per piece), so
    // in each of them the lane reads at the piece's first byte (1024 e, the
    // V^T image starting at piece K_PIECES) plus one per-lane offset, koff in
    // the K pieces and voff in the V^T pieces.
    static_assert(TF::K_PIECES % C8_WAVES == 0 && TF::PIECES % C8_WAVES == 0, "piece split");
    const uint32_t koff = [&] {
        const int row = wave * (512 / DK) + lane / TF::CPR;
        return (uint32_t)(2 * ((lane / TF::CPR) * DK + 8 * ((lane % TF::CPR) ^ TF::kswz(row))));
    }();
    const uint32_t voff = [&] {
        const int row = 4 * wave + (lane >> 4);
        return (uint32_t)(2 * ((lane >> 4) * FT_ROW + 8 * ((lane & 15) ^ (row & 15))));
    }();
    const unsigned char* src = reinterpret_cast<const unsigned char*>(
        p.tiles + (int64_t)bh * p.ntiles * TF::TILE);
    auto issue = [&](int tile) {
        // the history's last tile holds no keys when n_rows % 256 is in
        // (0, 128]: the decode never writes it and no step reads it
        if (tile < p.ntiles_hist && (int64_t)tile * FT_T >= p.n_rows) return;
        const unsigned char* s = src + (int64_t)tile * TF::TILE * 2;
        const int bi = (tile - t0) & 1;
        // opaque here, so that the per-piece sums are not hoisted out of
        // the tile loop into 64-bit registers: each load is a uniform base
        // plus the lane's 32-bit offset
        uint32_t ko = koff, vo = voff;
        asm volatile("" : "+v"(ko), "+v"(vo));
#pragma unroll
        for (int i = 0; i < TF::PIECES / C8_WAVES; ++i) {
            const int e = wave + C8_WAVES * i;
            if (i < TF::K_PIECES / C8_WAVES)
                dma16(s + 1024 * e + ko, sm.k[bi] + 512 * e);
            else
                dma16(s + 1024 * e + vo, sm.v[bi] + 512 * (e - TF::K_PIECES));
        }
    };
    const int hf = lane >> 5, l32 = lane & 31;
    const float c = p.scale_log2;
    using W = DWalk<DK>;
    constexpr int KS = W::KSTEPS;
    bf16x8 qf[KS], kf[KS], vf[8];
    const int64_t q0 = (int64_t)qb * 32;
    if (active) load_q_block<DK>(qf, p, b, h, q0, q0, lane);
    if (t0 < t1) issue(t0);
    // byte offsets in buffer 0 of this lane's operand fragments: K row l32
    // (+ 32 j) at its logical chunk of k-step kk, at chunk ^ kswz(l32); V^T
    // row l32 (+ 32 (t % 4)), logical chunk 4 j + 2 (t / 4) + hf, at
    // chunk ^ (l32 % 16)
    uint32_t kofs[KS], vofs[8];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        const int chunk = (W::block(kk) + W::HALF * hf) >> 3;
        kofs[kk] = 2 * (l32 * DK + 8 * (chunk ^ TF::kswz(l32)));
        asm volatile("" : "+v"(kofs[kk]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int chunk = 4 * (i >> 1) + 2 * (i & 1) + hf;
        vofs[i] = 2 * K_BYTES + 2 * (l32 * FT_ROW + 8 * (chunk ^ (l32 & 15)));
        asm volatile("" : "+v"(vofs[i]));
    }
    const uint32_t* mbase = nullptr;
    if (MASK && active) {
        const int64_t qi = min(q0 + l32, p.Q - 1);
        const int g = p.q_group ? min(max(p.q_group[qi], 0), p.n_groups - 1) : 0;
        mbase = p.cur_mask + (int64_t)g * p.mask_words;
    }
    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    // The softmax of one 32-key step's scores s and its P.V products with the
    // V^T fragments in vf (registers only).
    auto softmax_pv = [&](const f32x16& s) {
        float tm = fmaxf(s[0], s[1]);
#pragma unroll
        for (int i = 2; i < 16; ++i) tm = fmaxf(tm, s[i]);
        tm = halfwave_max(tm) * c;
        const bool up = tm > m + CK_TAU;
        const float mn = up ? tm : m;
        // m = -inf (nothing seen yet) gives alpha 0 on zero sums
        const float alpha = up ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
        m = mn;
        const float mref = MASK && mn == -INFINITY ? 0.0f : mn;
        uint32_t pw[8];
        float lsum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            pw[k] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(s[2 * k], c, -mref)),
                                __builtin_amdgcn_exp2f(fmaf(s[2 * k + 1], c, -mref)));
            lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[k]),
                                                   __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                                   lsum, false);
        }
        l = l * alpha + lsum;
        const bf16x8 p0 = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
        const bf16x8 p1 = as_bf16x8(u32x4{pw[4], pw[5], pw[6], pw[7]});
        __builtin_amdgcn_s_setprio(1);
        if (__any(up)) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = mfma32(vf[db], p0, o[db]);
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = mfma32(vf[4 + db], p1, o[db]);
        __builtin_amdgcn_s_setprio(0);
    };
    // Waves 4-7 run half a step behind waves 0-3 (wave w and w + 4 share a
    // SIMD): each carries its tile's last step (masked scores in s, V^T
    // fragments in vf) across the barrier and finishes it first in the next
    // tile.  On each SIMD one wave's softmax then overlaps the other's MFMA
    // products, instead of both waves reaching the same phase together after
    // every barrier.  Every wave still walks its steps in key order.
    const bool lag = wave >= C8_WAVES / 2;
    bool pend = false;
    f32x16 s;
    // The tiles in turn: kofs / vofs address the current tile's buffer and
    // move to the other one after each tile (uniform +-image size).
    for (int tile = t0; tile < t1; ++tile) {
        wait_loads_and_lds();
        __builtin_amdgcn_s_barrier();
        // the other buffer's last readers have passed the barrier (a carried
        // step holds its operands in registers)
        if (tile + 1 < t1) issue(tile + 1);
        const bool cur = tile >= p.ntiles_hist;
        const int64_t key0 = (int64_t)(cur ? tile - p.ntiles_hist : tile) * FT_T;
        const int valid = (int)min((int64_t)FT_T, (cur ? p.Nc : p.n_rows) - key0);
        const int nsub = active && valid > 0 ? (valid + 31) >> 5 : 0;
        auto lds_k = [&](int j, int kk) {
            return lds_b128(reinterpret_cast<const uint16_t*>(smem_raw + kofs[kk] + j * 32 * DK * 2));
        };
        auto lds_v = [&](int j, int t) {
            return lds_b128(reinterpret_cast<const uint16_t*>(
                smem_raw + vofs[2 * j + (t >> 2)] + (t & 3) * 32 * FT_ROW * 2));
        };
        // (an idle wave's reads of the first step stay inside the buffer)
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kf[kk] = lds_k(0, kk);
        if (pend) {
            softmax_pv(s);
            // the new tile's V^T reads wait for the carried products, so
            // that both fragment sets are never live at once
            __builtin_amdgcn_sched_barrier(0);
        }
        pend = false;
        const uint32_t* mrow = MASK && cur ? mbase + (key0 >> 5) : nullptr;
#pragma unroll
        for (int t = 0; t < 8; ++t) vf[t] = lds_v(0, t);
#pragma unroll
        for (int j = 0; j < FT_T / 32; ++j) {
            if (j >= nsub) break;
            __builtin_amdgcn_s_setprio(1);
            s = mfma32(kf[0], qf[0], f32x16{});
#pragma unroll
            for (int kk = 1; kk < KS; ++kk) s = mfma32(kf[kk], qf[kk], s);
            __builtin_amdgcn_s_setprio(0);
            if (j + 1 < nsub) {
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) kf[kk] = lds_k(j + 1, kk);
            }
            if (32 * j + 32 > valid) {
                const int vj = valid - 32 * j;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (8 * (i >> 2) + 4 * hf + (i & 3) >= vj) s[i] = -INFINITY;
            }
            if (MASK && cur) {
                const uint32_t bits = mrow[j];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (!((bits >> (8 * (i >> 2) + 4 * hf + (i & 3))) & 1u)) s[i] = -INFINITY;
            }
            if (lag && j + 1 == nsub) {
                pend = true;
                break;
            }
            softmax_pv(s);
            if (j + 1 < nsub) {
#pragma unroll
                for (int t = 0; t < 8; ++t) vf[t] = lds_v(j + 1, t);
            }
        }
        const int kstep = ((tile - t0) & 1) ? -K_BYTES : K_BYTES;
        const int vstep = ((tile - t0) & 1) ? -FT_IMG_BYTES : FT_IMG_BYTES;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            kofs[kk] += kstep;
            asm volatile("" : "+v"(kofs[kk]));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            vofs[i] += vstep;
            asm volatile("" : "+v"(vofs[i]));
        }
    }
    if (pend) softmax_pv(s);
    if (active) store_partial<false>(p, bh, split, q0, o, m, halfwave_sum(l), lane);
}

// The flash segments of a multi-partition launch.  Only a 128-wide
// partition has current keys, so MASK reaches that width alone.
template <bool MASK>
__global__ void __launch_bounds__(C8_THREADS, 1) flash8_kernel(MultiParams P) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int sg = multi_segment(P, blockIdx.x);
    const int pi = P.seg_part[sg], dk = P.dk[pi];
    const int64_t blk = (int64_t)blockIdx.x - P.seg_first[sg];
    if (dk == 32) flash_block<32, false>(P.part[pi], blk, smem_raw);
    else if (dk == 64) flash_block<64, false>(P.part[pi], blk, smem_raw);
    else flash_block<128, MASK>(P.part[pi], blk, smem_raw);
}

// Merge of chunk partials.  Two waves own one 32-query block, one per half
// of its 128 columns (lane-order rows 0-3 and 4-7 of the payload the
// attention wave stored, 1 KB per load instruction, four chunks in flight),
// and walk all its chunks; no cross-wave reduction, so blocks need no LDS.
// Both read the block's (m, l).
// out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c (O_c unnormalised); no
// chunks give out = 0 and lse = -inf (CN/core.py:48-49).
constexpr int CB_WAVES = 4;  // waves per 256-thread block
constexpr int CB_ROWS = 4;   // payload rows (of 8) per wave: half of the columns

// The running merge of one wave: M the largest chunk max so far, L the
// weighted row sum, acc the weighted O; Lx the part of L that the tracked
// source contributed (rescaled with L).
struct CombineAcc {
    float M, L, Lx;
    float acc[8 * CB_ROWS];
};

// Fold payload rows half * CB_ROWS .. +CB_ROWS of partials 0 .. NC of (bh,
// query block qblk) in, from a partial area of qblocks query blocks per
// (bh, chunk).  A chunk whose max exceeds M rescales the running sums (per
// lane), so no separate pass over the maxima delays the first partial loads.
__device__ __forceinline__ void combine_partials(CombineAcc& A, const uint16_t* part_o,
                                                 const float* part_ml, int64_t bh, int NC,
                                                 int qblocks, int qblk, int half, int lane,
                                                 bool track) {
    const int64_t qi = (int64_t)qblk * 32 + (lane & 31);
    const int64_t lse_stride = (int64_t)qblocks * 32;
    const u32x2* ml = reinterpret_cast<const u32x2*>(part_ml) + bh * NC * lse_stride + qi;
    const uint16_t* src = part_o + (bh * NC * qblocks + qblk) * 4096 + 512 * CB_ROWS * half + lane * 8;
    const int64_t cstride = (int64_t)qblocks * 4096;
    // a ring of CB_AHEAD chunks in flight (prefetches past the last chunk
    // reload it and are never used)
    constexpr int CB_AHEAD = 4;
    u32x4 buf[CB_AHEAD][CB_ROWS];
    u32x2 mlb[CB_AHEAD];
    auto issue = [&](int cc, int i) {
        cc = max(min(cc, NC - 1), 0);
        mlb[i] = ml[cc * lse_stride];
#pragma unroll
        for (int st = 0; st < CB_ROWS; ++st)
            buf[i][st] = *reinterpret_cast<const u32x4*>(src + cc * cstride + 512 * st);
        // chunks are issued in ring order, so waiting for slot i leaves the
        // slots issued after it in flight
        __builtin_amdgcn_sched_barrier(0);
    };
    // no chunks (no keys at all): nothing to read, and the workspace may be
    // null; the loads must not be issued ahead of this test
    if (NC <= 0) return;
    // fold slot i's chunk in (live: a chunk of this call, not a reload)
    auto fold = [&](int i, bool live) {
        const float mc = __uint_as_float(mlb[i][0]);
        // a chunk with no valid key for this query has m = -inf and O = 0
        const bool up = live && mc > A.M;
        if (__any(up)) {
            const float f = up ? exp2f(A.M - mc) : 1.0f;  // M = -inf gives 0
            A.L *= f;
            A.Lx *= f;
#pragma unroll
            for (int e = 0; e < 8 * CB_ROWS; ++e) A.acc[e] *= f;
        }
        A.M = up ? mc : A.M;
        const float wt = !live || mc == -INFINITY ? 0.0f : exp2f(mc - A.M);
        const float wl = wt * __uint_as_float(mlb[i][1]);
        A.L += wl;
        if (track) A.Lx += wl;
#pragma unroll
        for (int st = 0; st < CB_ROWS; ++st)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                A.acc[8 * st + 2 * e] += wt * __uint_as_float(buf[i][st][e] << 16);
                A.acc[8 * st + 2 * e + 1] += wt * __uint_as_float(buf[i][st][e] & 0xffff0000u);
            }
    };
    // up to CB_AHEAD chunks (the staged schedule's key splits): each loaded
    // once, all in flight before the first is folded in, and no reloads
    // that the wave would have to wait for before it ends
    auto fixed = [&](auto n) {
        constexpr int NF = decltype(n)::value;
#pragma unroll
        for (int i = 0; i < NF; ++i) issue(i, i);
#pragma unroll
        for (int i = 0; i < NF; ++i) fold(i, true);
    };
    if (NC == 1) return fixed(std::integral_constant<int, 1>{});
    if (NC == 2) return fixed(std::integral_constant<int, 2>{});
    if (NC == 3) return fixed(std::integral_constant<int, 3>{});
    if (NC == 4) return fixed(std::integral_constant<int, 4>{});
#pragma unroll
    for (int i = 0; i < CB_AHEAD; ++i) issue(i, i);
    for (int cc0 = 0; cc0 < NC; cc0 += CB_AHEAD) {
#pragma unroll
        for (int i = 0; i < CB_AHEAD; ++i) {
            // Slots past the last chunk hold a reloaded copy of it and get
            // weight 0.  No branch skips them, so the compiler's wait for
            // slot i leaves the other slots' loads in flight.
            fold(i, cc0 + i < NC);
            issue(cc0 + i + CB_AHEAD, i);
        }
    }
}

// Normalise and store this wave's half of query qi of (b, h): out = (acc +
// shift * Lx) / L in bf16 (shift: the row of 128 values added to the
// tracked source's output, or null), then, with ocam, bf16(P . out) for P
// of query row qi in the FULL layout (nkv_camera_apply's arithmetic); half
// 0 also writes lse = ln(sum) when lse is given.  With ocam both lanes of a
// query (lane and lane ^ 32, which hold the two halves of every 8-dim
// block) must reach this call.
__device__ __forceinline__ void combine_store(const CombineAcc& A, uint16_t* out, int64_t o_sb,
                                              int64_t o_st, int64_t o_sh, float* lse, int64_t Q,
                                              int H, int b, int h, int64_t qi, int half, int lane,
                                              const float* shift, const CameraDev* ocam = nullptr) {
    const int hf = lane >> 5;
    const float inv = A.L > 0.0f ? 1.0f / A.L : 0.0f;
    uint16_t* orow = out + b * o_sb + qi * o_st + h * o_sh + 4 * hf;
    // with ocam: rows 2 hf and 2 hf + 1 of P's four sub-frames for query qi,
    // rounded to bf16 once
    float pm[4][2][4];
    if (ocam) {
        const float* M = camera_mats(*ocam, b, qi);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const f32x4 m = ldg(reinterpret_cast<const f32x4*>(M + 16 * c + 4 * (2 * hf + r)));
#pragma unroll
                for (int e = 0; e < 4; ++e) pm[c][r][e] = bf16_round(m[e]);
            }
    }
    // acc[8*st + 2*e + {0,1}] (payload row st0 + st, st0 = CB_ROWS * half)
    // = o[db = st/2][i = 8*(st&1) + 2*e + {0,1}] with d = 32*db + 8*(i/4) +
    // 4*hf + i%4: acc[4n .. 4n+3] are four consecutive d of this lane's query
#pragma unroll
    for (int n = 0; n < 2 * CB_ROWS; ++n) {
        const int st = CB_ROWS * half + (n >> 1);
        const int db = st >> 1, i = 8 * (st & 1) + 4 * (n & 1);
        const int d = 32 * db + 8 * (i >> 2);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = A.acc[4 * n + e];
        if (shift) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = fmaf(shift[d + 4 * hf + e], A.Lx, v[e]);
        }
        u32x2 pk = {pack_bf16x2(v[0] * inv, v[1] * inv), pack_bf16x2(v[2] * inv, v[3] * inv)};
        if (ocam) {
            // block d / 8: this lane holds dims 4 hf .. 4 hf + 4, lane ^ 32 the
            // other four; its 4-vectors are the block's even and odd dims,
            // and this lane forms outputs 2 hf, 2 hf + 1 of each
            const uint32_t o0 = __shfl_xor(pk[0], 32), o1 = __shfl_xor(pk[1], 32);
            const uint32_t lo0 = hf ? o0 : pk[0], lo1 = hf ? o1 : pk[1];
            const uint32_t hi0 = hf ? pk[0] : o0, hi1 = hf ? pk[1] : o1;
            const float x0[4] = {__uint_as_float(lo0 << 16), __uint_as_float(lo1 << 16),
                                 __uint_as_float(hi0 << 16), __uint_as_float(hi1 << 16)};
            const float x1[4] = {__uint_as_float(lo0 & 0xffff0000u), __uint_as_float(lo1 & 0xffff0000u),
                                 __uint_as_float(hi0 & 0xffff0000u), __uint_as_float(hi1 & 0xffff0000u)};
            const int c = (d >> 3) & 3;
            float y[2][2];
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    // camera_vec4's sum for one output, the products exact
#pragma clang fp contract(off)
                    double acc = 0.0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc += (double)(pm[c][r][e] * (v ? x1[e] : x0[e]));
                    y[r][v] = bf16_round(f64_to_f32(acc));
                }
            pk = {pack_bf16x2(y[0][0], y[0][1]), pack_bf16x2(y[1][0], y[1][1])};
        }
        *reinterpret_cast<u32x2*>(orow + d) = pk;
    }
    if (lse && hf == 0 && half == 0)
        lse[((int64_t)b * H + h) * Q + qi] =
            A.L > 0.0f ? (A.M + log2f(A.L)) * 0.69314718055994531f : -INFINITY;
}

__device__ __forceinline__ void combine_init(CombineAcc& A) {
    A.M = -INFINITY;
    A.L = A.Lx = 0.0f;
#pragma unroll
    for (int e = 0; e < 8 * CB_ROWS; ++e) A.acc[e] = 0.0f;
}

// The key-chunk schedule's merge: every (b, h, q) of one launch.
__global__ void __launch_bounds__(64 * CB_WAVES) chunk_combine_kernel(ChunkParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t gw = (int64_t)blockIdx.x * CB_WAVES + wave;
    const int64_t gq = gw >> 1;
    const int half = (int)(gw & 1);
    if (gq >= (int64_t)p.B * p.H * p.qblocks) return;
    const int64_t bh = gq / p.qblocks;
    const int qblk = (int)(gq % p.qblocks);
    CombineAcc A;
    combine_init(A);
    combine_partials(A, p.part_o, p.part_ml, bh, p.nch_total, p.qblocks, qblk, half, lane, false);
    const int64_t qi = (int64_t)qblk * 32 + (lane & 31);
    if (qi >= p.Q) return;
    combine_store(A, p.out, p.o_sb, p.o_st, p.o_sh, p.lse, p.Q, p.H, (int)(bh / p.H),
                  (int)(bh % p.H), qi, half, lane, nullptr);
}

// The staged schedule's merge over every partition (CN/core.py:33-42 for
// two): one wave per (b, h, query block) of partition 0, which covers every
// head of the layer, folds in that head's partials of partition 0, then of
// the first other partition that lists h among its heads, whose output is
// shifted by shift[b*sh_sb + h*sh_sh + d] (null: none; the value-mean
// correction) before the merge.
__global__ void __launch_bounds__(64 * CB_WAVES) staged_combine_kernel(MultiParams P,
                                                                       const float* shift,
                                                                       int64_t sh_sb, int64_t sh_sh,
                                                                       CameraDev ocam) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const ChunkParams& n = P.part[0];
    const int64_t gw = (int64_t)blockIdx.x * CB_WAVES + wave;
    const int64_t gq = gw >> 1;
    const int half = (int)(gw & 1);
    if (gq >= (int64_t)n.B * n.H * n.qblocks) return;
    const int64_t bh = gq / n.qblocks;
    const int qblk = (int)(gq % n.qblocks);
    const int b = (int)(bh / n.H), h = (int)(bh % n.H);
    // the partition holding head h besides partition 0 (0: none)
    int lp = 0, li = 0;
    for (int pi = 1; pi < NKV_MAX_PARTS && pi < P.nparts && lp == 0; ++pi)
        for (int i = 0; i < P.part[pi].H; ++i)
            if (ldg(P.heads[pi] + i) == h) {
                lp = pi;
                li = i;
                break;
            }
    CombineAcc A;
    combine_init(A);
    for (int src = 0; src < (lp ? 2 : 1); ++src) {
        const ChunkParams& g = P.part[src ? lp : 0];
        combine_partials(A, g.part_o, g.part_ml, src ? (int64_t)b * g.H + li : bh, g.nch_total,
                         g.qblocks, qblk, half, lane, src == 1);
    }
    const int64_t qi = (int64_t)qblk * 32 + (lane & 31);
    if (qi >= n.Q) return;
    combine_store(A, n.out, n.o_sb, n.o_st, n.o_sh, n.lse, n.Q, n.H, b, h, qi, half, lane,
                  lp && shift ? shift + (int64_t)b * sh_sb + (int64_t)h * sh_sh : nullptr,
                  ocam.mats ? &ocam : nullptr);
}

// ------------------------------------------------------------------ host
ChunkCodec chunk_codec_from(const nkv_codec& c, int D, int HD) {
    ChunkCodec v{};
    v.r = c.r;
    v.group = c.group;
    v.scale_dtype = c.scale_dtype;
    v.w = c.w_dec;
    v.w_hs = (int64_t)D * c.r;
    v.c_rs = HD;
    v.c_hs = D;
    v.bias = c.mean;
    v.bias_hs = D;
    if (c.n_segments > 0) {
        // each segment's own table (checked on the host: all or none have one)
        v.seg = c.segments_dev;
        v.n_seg = c.n_segments;
        v.seg_flat = 0;
        v.has_centers = c.segments[0].centers != nullptr;
        return v;
    }
    v.packed = c.packed;
    v.scales = c.scales;
    v.ids = c.centers ? c.ids : nullptr;
    v.id_bytes = c.id_bytes;
    v.num_centers = c.num_centers;
    v.centers = c.centers;
    v.c_bs = c.centers_batch_stride;
    v.has_centers = c.centers != nullptr;
    return v;
}

int check_segments(const nkv_codec& c, int64_t N) {
    if (c.n_segments == 0) return NKV_OK;
    NKV_REQUIRE(c.n_segments > 0 && c.segments && c.segments_dev, NKV_ERR_INVALID,
                "a segmented codec needs its host and device segment tables");
    const bool cent = c.segments[0].centers != nullptr;
    int64_t row = 0, cbase = 0;
    for (int i = 0; i < c.n_segments; ++i) {
        const nkv_segment& s = c.segments[i];
        NKV_REQUIRE(s.packed && s.scales && s.rows >= 1, NKV_ERR_INVALID,
                    "every segment needs packed codes, scales and at least one row");
        NKV_REQUIRE(s.row_start == row, NKV_ERR_INVALID,
                    "segments must be in row order and contiguous from row 0");
        NKV_REQUIRE((s.centers != nullptr) == cent, NKV_ERR_INVALID,
                    "every segment must have a center table, or none");
        if (cent) {
            NKV_REQUIRE(s.ids && (s.id_bytes == 1 || s.id_bytes == 2 || s.id_bytes == 4) &&
                            s.num_centers > 0 && s.centers_batch_stride >= 0,
                        NKV_ERR_INVALID, "segment centers need ids of 1, 2 or 4 bytes");
            NKV_REQUIRE(s.center_base == cbase, NKV_ERR_INVALID,
                        "segment center_base must be the sum of the tables before it");
            cbase += s.num_centers;
        }
        row += s.rows;
    }
    NKV_REQUIRE(row == N, NKV_ERR_INVALID, "the segments must hold exactly the codec's N rows");
    return NKV_OK;
}

namespace {

int64_t chunk_count(int64_t keys) { return cdiv(keys, CK_T); }

int check_chunk_codec(const ChunkCodec& c) {
    NKV_REQUIRE((c.seg || (c.packed && c.scales)) && c.w, NKV_ERR_INVALID,
                "history codec needs packed codes, scales and decode rows");
    NKV_REQUIRE(c.r > 0 && c.r % 64 == 0 && c.r <= 4096, NKV_ERR_UNSUPPORTED,
                "key-chunk attend needs codec ranks that are multiples of 64");
    NKV_REQUIRE(c.group > 0 && c.group % 32 == 0 && c.r % c.group == 0, NKV_ERR_UNSUPPORTED,
                "key-chunk attend needs scale groups that are multiples of 32 dividing r");
    NKV_REQUIRE(c.scale_dtype == NKV_DTYPE_BF16 || c.scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    if (c.has_centers && !c.seg) {
        NKV_REQUIRE(c.centers && c.ids && (c.id_bytes == 1 || c.id_bytes == 2 || c.id_bytes == 4),
                    NKV_ERR_INVALID, "centers need ids of 1, 2 or 4 bytes");
        NKV_REQUIRE(c.num_centers > 0, NKV_ERR_INVALID, "num_centers must be > 0");
    }
    NKV_REQUIRE(!c.seg || c.n_seg > 0, NKV_ERR_INVALID, "empty segment table");
    NKV_REQUIRE(!(c.seg && c.has_centers && c.seg_flat) || c.centers, NKV_ERR_INVALID,
                "a flat center table is missing");
    NKV_REQUIRE(!c.c_heads || c.c_heads_n >= 1, NKV_ERR_INVALID, "c_heads needs c_heads_n >= 1");
    return NKV_OK;
}

template <int DK, bool MASK>
void launch_dk(const ChunkParams& p, int64_t blocks, hipStream_t s, int* rc) {
    const size_t smem = sizeof(Chunk8Smem);
    hipError_t e = hipFuncSetAttribute((const void*)chunk8_kernel<DK, MASK>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
        set_error(std::string("chunk_launch: hipFuncSetAttribute failed: ") + hipGetErrorString(e));
        *rc = NKV_ERR_HIP;
        return;
    }
    chunk8_kernel<DK, MASK><<<dim3((unsigned)blocks), C8_THREADS, smem, s>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string("chunk_launch: launch failed: ") + hipGetErrorString(e));
        *rc = NKV_ERR_HIP;
    }
}

template <typename K>
int set_smem(K* kernel, size_t smem) {
    const hipError_t e = hipFuncSetAttribute((const void*)kernel,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
        set_error(std::string("chunk_launch: hipFuncSetAttribute failed: ") + hipGetErrorString(e));
        return NKV_ERR_HIP;
    }
    return NKV_OK;
}

// ---------------------------------------------------------- staged (host)
constexpr int FT_CUS = 256;          // compute units of an MI355X
// The staged schedule from one query block up.  Measured on MI355X against
// the key-chunk kernel (cfg1's codec, 24 heads, Q = Nc), the staged call was
// faster at every size tried: 1 block over 49,920 history keys 0.543 vs
// 0.571 ms, over 12,480 keys 0.161 vs 0.177 ms; 6 blocks 0.590 vs 0.660 and
// 0.174 vs 0.202 ms; 12 blocks 0.747 vs 0.837 and 0.224 vs 0.254 ms; cfg2 (25
// blocks) 0.950 vs 1.067 ms.  The key-chunk kernel remains for reader widths
// 32/64 with ranks above 384 (read-time RoPE and the FULL camera layout are
// tile_xform_kernel's pass over the decoded tiles).
constexpr int FT_MIN_QBLOCKS = 1;

struct FlashPlan {
    int qpt, qtiles, splits, ntiles_hist, ntiles;
};

// Query tiles of at most eight blocks, balanced (49 blocks: 7 tiles of 7).
FlashPlan flash_shape(const ChunkLaunchDesc& d) {
    FlashPlan f{};
    const int64_t qblocks = cdiv(d.Q, 32);
    f.qtiles = (int)cdiv(qblocks, C8_WAVES);
    f.qpt = (int)cdiv(qblocks, f.qtiles);
    f.ntiles_hist = 2 * (int)chunk_count(d.n_rows);
    f.ntiles = f.ntiles_hist + 2 * (int)chunk_count(d.Nc);
    f.splits = 0;
    return f;
}

// History tiles from the decode GEMM with the decoder held in LDS (the
// current tiles copied in the same launch; read-time RoPE and the camera's
// FULL layout applied by tile_xform_kernel); with the SF13 camera layout, or
// ranks above what LDS holds, both from stage8_kernel's decode.
bool staged_gemm(const ChunkLaunchDesc& d) {
    return (!d.cam.mats || d.cam.layout == NKV_CAMERA_FULL) && d.key.r <= 64 * DR_MAXQ &&
           d.value.r <= 64 * DR_MAXQ;
}

// Reader widths below 128 are staged only by the decode GEMM (stage8_kernel
// decodes at full width).
bool use_staged(const ChunkLaunchDesc& d) {
    const bool width = d.dk == CK_D || ((d.dk == 32 || d.dk == 64) && staged_gemm(d));
    return width && cdiv(d.Q, 32) >= FT_MIN_QBLOCKS && d.n_rows + d.Nc > 0;
}

// Cost model of the staged kernels for planning their grids, in units of one
// 128-wide tile of a kernel's steady state (on MI355X the flash kernel takes
// ~4.4 us per tile and block at 128 wide, ~3.1 us at 32; the decode ~5 us),
// plus a fixed cost per block (the decode's: the decoder rows and the
// range's center rows, ~8 us).
double flash_tile_cost(int dk) { return dk == 32 ? 0.7 : dk == 64 ? 0.82 : 1.0; }
// Modelled costs in units of one 128-wide K tile's decode (about 4.4 us of
// a decode block at cfg1): a V tile (the centers' loads and adds in the
// accumulator layout) 1.1; a decode block's start (the decoder rows of all
// blocks load at once) DECODE_BLOCK_COST, and each further head piece of it
// (its decoder rows, bias and center references again) DECODE_PIECE_COST;
// one batch of CJ_BATCH current tiles of a current-key block
// CTILE_BATCH_COST (about 12 us).
double decode_tile_cost(int w, int cc) {
    return cc ? 1.1 : w == 32 ? 0.5 : w == 64 ? 0.7 : 1.0;
}
constexpr double FLASH_BLOCK_COST = 1.0, DECODE_BLOCK_COST = 2.0, DECODE_PIECE_COST = 0.75,
                 CTILE_BATCH_COST = 2.7;
constexpr double FLASH_TILE_US = 4.4;
// each split's partials are written by the flash kernel and read back by the
// combine at about 4 TB/s
constexpr double PARTIAL_BYTES_PER_US = 4.0e6;
constexpr size_t PARTIAL_ROW_BYTES = CK_D * sizeof(uint16_t) + 2 * sizeof(float);

// Finishing time of greedy list scheduling (largest blocks first, each to
// the least loaded CU) of groups of equal blocks (cost, count) on FT_CUS
// CUs.  CUs with equal loads are kept as one entry, so each step places a
// whole run of blocks.
double lpt_makespan(std::vector<std::pair<double, int64_t>> groups) {
    std::sort(groups.begin(), groups.end(),
              [](const std::pair<double, int64_t>& x, const std::pair<double, int64_t>& y) {
                  return x.first > y.first;
              });
    std::map<double, int64_t> loads{{0.0, FT_CUS}};
    double span = 0.0;
    for (const auto& g : groups) {
        int64_t n = g.second;
        while (n > 0) {
            auto it = loads.begin();
            const double at = it->first;
            const int64_t take = std::min(n, it->second);
            if (take == it->second) loads.erase(it);
            else it->second -= take;
            loads[at + g.first] += take;
            span = std::max(span, at + g.first);
            n -= take;
        }
    }
    return span;
}

// The staged plan of partitions d[0 .. n): flash key splits per partition,
// decode tile ranges per (partition, codec), the workspace layout.
struct MultiPlan {
    int n;
    FlashPlan f[NKV_MAX_PARTS];
    int dblocks[NKV_MAX_PARTS][2];  // decode blocks of K and V (0: no history)
    int cblocks[NKV_MAX_PARTS];     // current-key blocks (0: no current keys)
    size_t tiles_off[NKV_MAX_PARTS], part_off[NKV_MAX_PARTS];
    // each camera partition's fp64 matrix table (after every tile and
    // partial area, which end at areas_end)
    size_t cam_off[NKV_MAX_PARTS], areas_end, total;
};

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Bytes of a partition's fp64 camera table: the staged decode GEMM's tile
// pass reads the matrices from it (0: no camera on that path).
int64_t cam_table_bytes(const ChunkLaunchDesc& d) {
    if (!d.cam.mats || !staged_gemm(d)) return 0;
    return (int64_t)camera_batches(d.cam, d.B) * d.cam.n_mats * 64 * (int64_t)sizeof(double);
}

// Key splits: every split count of every partition gives a candidate block
// cost; each candidate gives each partition the fewest splits whose blocks
// stay within it, and the plan with the least modelled time (the makespan
// plus the partials' traffic) wins.  One partition at cfg1 (112 tiles, 168
// query tiles): 3 splits, 504 blocks in two rounds of the CUs.
void plan_flash(const ChunkLaunchDesc* d, int n, MultiPlan& P) {
    std::vector<double> cand;
    double work[NKV_MAX_PARTS];
    int smax[NKV_MAX_PARTS];
    for (int i = 0; i < n; ++i) {
        P.f[i] = flash_shape(d[i]);
        work[i] = P.f[i].ntiles * flash_tile_cost(d[i].dk);
        smax[i] = std::max(1, std::min(16, P.f[i].ntiles / 4));
        if (P.f[i].ntiles == 0) continue;
        for (int sp = 1; sp <= smax[i]; ++sp) cand.push_back(work[i] / sp);
    }
    double best = 1e300;
    int64_t best_blocks = 0;
    int best_sp[NKV_MAX_PARTS] = {};
    for (const double c : cand) {
        std::vector<std::pair<double, int64_t>> groups;
        int sp[NKV_MAX_PARTS] = {};
        int64_t blocks = 0;
        double bytes = 0.0;
        for (int i = 0; i < n; ++i) {
            if (P.f[i].ntiles == 0) continue;
            sp[i] = std::min(smax[i], std::max(1, (int)std::ceil(work[i] / c - 1e-9)));
            const int64_t nb = (int64_t)d[i].B * d[i].H * P.f[i].qtiles * sp[i];
            groups.push_back({work[i] / sp[i] + FLASH_BLOCK_COST, nb});
            blocks += nb;
            bytes += 2.0 * (double)d[i].B * d[i].H * sp[i] * cdiv(d[i].Q, 32) * 32 * PARTIAL_ROW_BYTES;
        }
        const double t = lpt_makespan(groups) * FLASH_TILE_US + bytes / PARTIAL_BYTES_PER_US;
        if (t < best - 1e-6 || (t < best + 1e-6 && blocks < best_blocks)) {
            best = t;
            best_blocks = blocks;
            for (int i = 0; i < n; ++i) best_sp[i] = sp[i];
        }
    }
    for (int i = 0; i < n; ++i) P.f[i].splits = best_sp[i];
}

// Decode blocks: each (partition, codec) segment's B*H*T history tiles in nb
// equal ranges (nb a multiple of 8, no range above DR_MAXT tiles); a block
// pays a head piece per head its range touches, B*H / nb more than one on
// average.
// Current-key blocks: a pool of them builds every partition's current tiles
// in batches (each partition's share in proportion to its tiles), sized to
// the CUs the decode blocks leave free or to one batch per block.  Candidate
// per-block decode costs come from every segment's choices of nb (up to two
// rounds of the CUs); the plan with the least modelled makespan (fewest
// blocks on ties) wins.  cfg1 (24 heads, 98 history and 13 current tiles per
// head): 112 K and 128 V blocks, 16 current-key blocks of 5 batches.
void plan_decode(const ChunkLaunchDesc* d, int n, MultiPlan& P) {
    struct Seg {
        int i, cc;
        int64_t bh, nmin, nmax;
        double w;
    };
    auto round8 = [](int64_t x) { return 8 * cdiv(x, 8); };
    std::vector<Seg> segs;
    int64_t jobs[NKV_MAX_PARTS] = {}, all_jobs = 0;
    for (int i = 0; i < n; ++i) {
        P.dblocks[i][0] = P.dblocks[i][1] = 0;
        P.cblocks[i] = 0;
        const int64_t bh = (int64_t)d[i].B * d[i].H;
        jobs[i] = bh * (P.f[i].ntiles - P.f[i].ntiles_hist);
        all_jobs += jobs[i];
        if (d[i].n_rows > 0) {
            const int64_t M = bh * cdiv(d[i].n_rows, FT_T);
            const int64_t nmin = round8(cdiv(M, DR_MAXT));
            const int64_t nmax = std::max(nmin, round8(std::min(M, (int64_t)2 * FT_CUS)));
            for (int cc = 0; cc < 2; ++cc)
                segs.push_back({i, cc, bh, nmin, nmax, M * decode_tile_cost(d[i].dk, cc)});
        }
    }
    // the current-key pool of `pool` blocks over the partitions
    auto share = [&](int64_t pool, int64_t (&c)[NKV_MAX_PARTS]) {
        for (int i = 0; i < n; ++i)
            c[i] = jobs[i] ? std::min(jobs[i], std::max((int64_t)1, pool * jobs[i] / all_jobs)) : 0;
    };
    auto add_cur = [&](std::vector<std::pair<double, int64_t>>& groups, const int64_t (&c)[NKV_MAX_PARTS]) {
        int64_t blocks = 0;
        for (int i = 0; i < n; ++i)
            if (c[i]) {
                groups.push_back({(double)cdiv(cdiv(jobs[i], c[i]), CJ_BATCH) * CTILE_BATCH_COST, c[i]});
                blocks += c[i];
            }
        return blocks;
    };
    auto block_cost = [](const Seg& g, int64_t nb) {
        return g.w / nb + DECODE_BLOCK_COST + DECODE_PIECE_COST * (double)g.bh / nb;
    };
    std::vector<double> cand;
    for (const Seg& g : segs)
        for (int64_t nb = g.nmin; nb <= g.nmax; nb += 8) cand.push_back(g.w / nb);
    if (cand.empty()) cand.push_back(1.0);  // current keys only
    // K and V decode in separate launches when their ranks differ (the
    // current keys with K): the makespans add
    const bool split = (d[0].key.r >> 6) != (d[0].value.r >> 6);
    double best = 1e300;
    int64_t best_blocks = 0;
    std::vector<int64_t> best_nb(segs.size()), nb(segs.size());
    int64_t best_c[NKV_MAX_PARTS] = {};
    for (const double c : cand) {
        std::vector<std::pair<double, int64_t>> dec[2];
        int64_t dblocks = 0, first_launch = 0;
        for (size_t k = 0; k < segs.size(); ++k) {
            const Seg& g = segs[k];
            nb[k] = std::min(g.nmax, std::max(g.nmin, round8((int64_t)std::ceil(g.w / c - 1e-9))));
            dec[split ? g.cc : 0].push_back({block_cost(g, nb[k]), nb[k]});
            dblocks += nb[k];
            if (!split || g.cc == 0) first_launch += nb[k];
        }
        const int64_t pools[2] = {std::max((int64_t)8, FT_CUS - first_launch), cdiv(all_jobs, CJ_BATCH)};
        for (int q = 0; q < (all_jobs ? 2 : 1); ++q) {
            int64_t cb[NKV_MAX_PARTS];
            share(pools[q], cb);
            std::vector<std::pair<double, int64_t>> groups = dec[0];
            const int64_t blocks = dblocks + add_cur(groups, cb);
            const double t = lpt_makespan(groups) + (split ? lpt_makespan(dec[1]) : 0.0);
            if (t < best - 1e-6 || (t < best + 1e-6 && blocks < best_blocks)) {
                best = t;
                best_blocks = blocks;
                best_nb = nb;
                for (int i = 0; i < n; ++i) best_c[i] = cb[i];
            }
        }
    }
    for (size_t k = 0; k < segs.size(); ++k) P.dblocks[segs[k].i][segs[k].cc] = (int)best_nb[k];
    for (int i = 0; i < n; ++i) P.cblocks[i] = (int)best_c[i];
}

// The byte extents the staged kernels write in a plan's workspace, checked
// against each partition's slice [tiles_off, part_off) of tile images and
// [part_off, next tiles_off) of split partials: the last tile's V^T image as
// the decode addresses it (tile t of head bh at (bh * ntiles + t) tile
// images, its V^T image after the K image, both at the partition's width;
// v_dk != 0 addresses the V^T images at that width instead, to check a
// layout mismatch), the current tiles' copies (128 wide) and the flash
// kernel's partials (a 32 x 128 bf16 block per (b*h, split, query block),
// then (m, l) per query).  On a violation, msg names it.
bool plan_extents_ok(const MultiPlan& P, const ChunkLaunchDesc* d, int n, int v_dk,
                     std::string* msg) {
    for (int i = 0; i < n; ++i) {
        const FlashPlan& f = P.f[i];
        const size_t bh = (size_t)d[i].B * d[i].H;
        const size_t tile = tile_elems(d[i].dk) * sizeof(uint16_t);
        const size_t slice_end = P.part_off[i];
        const size_t tiles_end = P.tiles_off[i] + bh * f.ntiles * tile;
        auto fail = [&](const char* what, size_t end, size_t lim) {
            if (msg)
                *msg = "partition " + std::to_string(i) + " (width " + std::to_string(d[i].dk) +
                       "): " + what + " ends at byte " + std::to_string(end) + ", past " +
                       std::to_string(lim);
            return false;
        };
        if (tiles_end > slice_end) return fail("tile images", tiles_end, slice_end);
        const int64_t hist = cdiv(d[i].n_rows, FT_T);
        if (hist > 0 && bh > 0) {
            const int vw = v_dk ? v_dk : d[i].dk;
            const size_t vtile = tile_elems(vw) * sizeof(uint16_t);
            const size_t v_end = P.tiles_off[i] + ((bh - 1) * f.ntiles + hist - 1) * vtile +
                                 (k_image_elems(vw) + FT_IMG) * sizeof(uint16_t);
            if (v_end > tiles_end) return fail("the last V^T image", v_end, tiles_end);
        }
        if (f.ntiles > f.ntiles_hist && d[i].dk != CK_D)
            return fail("current tiles at a width other than 128", tiles_end, tiles_end);
        // the decode launch's blocks: equal ranges of at most DR_MAXT tiles
        // per codec (a multiple of 8 blocks), and current-key blocks whenever
        // there are current tiles
        if (staged_gemm(d[i])) {
            auto bad = [&](const std::string& what) {
                if (msg) *msg = "partition " + std::to_string(i) + ": " + what;
                return false;
            };
            for (int cc = 0; cc < 2 && hist > 0; ++cc) {
                const int nb = P.dblocks[i][cc];
                if (nb <= 0 || nb % 8 || cdiv((int64_t)bh * hist, nb) > DR_MAXT)
                    return bad("decode blocks " + std::to_string(nb) + " for " +
                               std::to_string((int64_t)bh * hist) + " tiles");
            }
            if (f.ntiles > f.ntiles_hist && P.cblocks[i] <= 0)
                return bad("current tiles without current-key blocks");
        }
        const size_t rows = bh * f.splits * cdiv(d[i].Q, 32) * 32;
        const size_t part_end = P.part_off[i] + rows * PARTIAL_ROW_BYTES;
        const size_t lim = i + 1 < n ? P.tiles_off[i + 1] : P.areas_end;
        if (part_end > lim) return fail("the split partials", part_end, lim);
    }
    return true;
}

// The plan depends on the partitions' shapes and codec ranks alone; the last
// one is kept (a layer loop repeats the same shapes).
MultiPlan multi_plan(const ChunkLaunchDesc* d, int n) {
    std::vector<int64_t> key{n};
    for (int i = 0; i < n; ++i)
        for (int64_t v : {(int64_t)d[i].B, (int64_t)d[i].H, (int64_t)d[i].dk, d[i].Q, d[i].n_rows,
                          d[i].Nc, (int64_t)staged_gemm(d[i]), cam_table_bytes(d[i]),
                          (int64_t)d[i].key.r, (int64_t)d[i].value.r})
            key.push_back(v);
    thread_local std::vector<int64_t> last_key;
    thread_local MultiPlan last;
    if (key == last_key) return last;
    MultiPlan P{};
    P.n = n;
    plan_flash(d, n, P);
    plan_decode(d, n, P);
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        const FlashPlan& f = P.f[i];
        P.tiles_off[i] = off;
        off += align256((size_t)d[i].B * d[i].H * f.ntiles * tile_elems(d[i].dk) * sizeof(uint16_t));
        P.part_off[i] = off;
        off += align256((size_t)d[i].B * d[i].H * f.splits * cdiv(d[i].Q, 32) * 32 * PARTIAL_ROW_BYTES);
    }
    P.areas_end = off;
    for (int i = 0; i < n; ++i) {
        P.cam_off[i] = off;
        off += align256((size_t)cam_table_bytes(d[i]));
    }
    P.total = off;
    last_key = key;
    last = P;
    return P;
}

template <int KQ>
int drtile_launch_kq(const MultiParams& M, int64_t blocks, hipStream_t s) {
    const int rc = set_smem(drtile_kernel<KQ>, sizeof(DResSmem));
    if (rc) return rc;
    drtile_kernel<KQ><<<dim3((unsigned)blocks), DR_THREADS, sizeof(DResSmem), s>>>(M);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

int drtile_launch(int kq, const MultiParams& M, int64_t blocks, hipStream_t s) {
    switch (kq) {
        case 1: return drtile_launch_kq<1>(M, blocks, s);
        case 2: return drtile_launch_kq<2>(M, blocks, s);
        case 3: return drtile_launch_kq<3>(M, blocks, s);
        case 4: return drtile_launch_kq<4>(M, blocks, s);
        case 5: return drtile_launch_kq<5>(M, blocks, s);
        default: return drtile_launch_kq<6>(M, blocks, s);
    }
}

// Block cost of a segment for ordering a launch (largest first).
struct SegOrder {
    double cost;
    int part, kind, ranges;
    int64_t blocks;
};

void set_segments(MultiParams& M, std::vector<SegOrder> segs) {
    std::stable_sort(segs.begin(), segs.end(),
                     [](const SegOrder& x, const SegOrder& y) { return x.cost > y.cost; });
    M.nseg = (int)segs.size();
    int64_t first = 0;
    for (int k = 0; k < M.nseg; ++k) {
        M.seg_part[k] = segs[k].part;
        M.seg_kind[k] = segs[k].kind;
        M.seg_ranges[k] = segs[k].ranges;
        M.seg_first[k] = first;
        first += segs[k].blocks;
    }
    for (int k = M.nseg; k <= MP_SEGS; ++k) M.seg_first[k] = first;
}

int64_t seg_blocks(const MultiParams& M) { return M.seg_first[M.nseg]; }

// Stage, flash, combine of partitions d[0 .. n); ps[i] holds everything of
// partition i but the staged fields.
int staged_run(hipStream_t s, const ChunkLaunchDesc* d, const ChunkParams* ps, int n,
               const int32_t* const* heads, const float* shift, int64_t sh_sb, int64_t sh_sh,
               void* workspace, const CameraDev& ocam = CameraDev{}) {
    const MultiPlan P = multi_plan(d, n);
    {
        std::string why;
        NKV_REQUIRE(plan_extents_ok(P, d, n, 0, &why), NKV_ERR_INVALID,
                    "internal: staged workspace plan: " + why);
    }
    NKV_REQUIRE(staged_gemm(d[0]) || (n == 1 && d[0].dk == CK_D), NKV_ERR_INVALID,
                "internal: stage8_kernel decodes one 128-wide partition");
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    MultiParams M;
    memset(&M, 0, sizeof(M));
    M.nparts = n;
    for (int i = 0; i < n; ++i) {
        const FlashPlan& f = P.f[i];
        ChunkParams p = ps[i];
        p.tiles = reinterpret_cast<uint16_t*>(ws + P.tiles_off[i]);
        p.ntiles_hist = f.ntiles_hist;
        p.ntiles = f.ntiles;
        p.qpt = f.qpt;
        p.qtiles = f.qtiles;
        p.splits = std::max(f.splits, 1);
        // the partials of the splits, in the key-chunk layout with chunk = split
        p.nch_hist = 0;
        p.nch_total = f.splits;
        p.part_o = reinterpret_cast<uint16_t*>(ws + P.part_off[i]);
        p.part_ml = reinterpret_cast<float*>(
            p.part_o + (size_t)d[i].B * d[i].H * f.splits * p.qblocks * 32 * CK_D);
        M.part[i] = p;
        M.dk[i] = d[i].dk;
        M.heads[i] = heads ? heads[i] : nullptr;
    }
    int rc = NKV_OK;
    // the fp64 matrix table of each camera of the tile pass, once per
    // distinct camera (filled by the decode launch, table[i] set)
    bool table[NKV_MAX_PARTS] = {};
    for (int i = 0; i < n; ++i) {
        if (!cam_table_bytes(d[i])) continue;
        CameraDev& c = M.part[i].cam;
        for (int k = 0; k < i && !c.m64; ++k) {
            const CameraDev& o = M.part[k].cam;
            if (o.m64 && o.mats == c.mats && o.mats_bs == c.mats_bs && o.n_mats == c.n_mats &&
                d[k].B == d[i].B)
                c.m64 = o.m64;
        }
        if (c.m64) continue;
        c.m64 = reinterpret_cast<const double*>(ws + P.cam_off[i]);
        table[i] = true;
    }
    if (!staged_gemm(d[0])) {
        // one partition at width 128 with the SF13 camera layout, or ranks
        // above the resident decoder's: stage8_kernel decodes its history and
        // current tiles
        const ChunkParams& p = M.part[0];
        rc = set_smem(stage8_kernel, sizeof(Chunk8Smem));
        if (rc) return rc;
        stage8_kernel<<<dim3((unsigned)((int64_t)d[0].B * d[0].H * P.f[0].ntiles / 2)), C8_THREADS,
                        sizeof(Chunk8Smem), s>>>(p);
        NKV_LAUNCH_CHECK();
    } else {
        // both codecs in one launch when their ranks agree, the current
        // tiles with the first
        const int qk = d[0].key.r >> 6, qv = d[0].value.r >> 6;
        for (int pass = 0; pass < (qk == qv ? 1 : 2); ++pass) {
            std::vector<SegOrder> segs;
            for (int i = 0; i < n; ++i) {
                const int64_t bh = (int64_t)d[i].B * d[i].H;
                const int64_t T = cdiv(d[i].n_rows, FT_T);
                for (int cc = 0; cc < 2; ++cc) {
                    const int nb = P.dblocks[i][cc];
                    if (nb == 0 || (qk != qv && cc != pass)) continue;
                    // ordered by block cost, before the current-key and
                    // table segments (cost 0), so each starts at a
                    // multiple of 8
                    segs.push_back({(double)bh * T / nb * decode_tile_cost(d[i].dk, cc) + DECODE_BLOCK_COST,
                                    i, cc ? SEG_V : SEG_K, nb, nb});
                }
                if (pass == 0 && P.cblocks[i] > 0)
                    segs.push_back({0.0, i, SEG_CUR, P.cblocks[i], P.cblocks[i]});
                if (pass == 0 && table[i]) {
                    const CameraDev& c = M.part[i].cam;
                    const int64_t elems = (int64_t)camera_batches(c, d[i].B) * c.n_mats * 64;
                    segs.push_back({0.0, i, SEG_TABLE, 0, cdiv(elems, DR_THREADS)});
                }
            }
            set_segments(M, segs);
            if (seg_blocks(M) == 0) continue;
            rc = drtile_launch(qk == qv || pass == 0 ? qk : qv, M, seg_blocks(M), s);
            if (rc) return rc;
        }
        // read-time RoPE and the camera of every partition's history tiles,
        // in place
        std::vector<SegOrder> segs;
        for (int i = 0; i < n; ++i)
            if ((rope_on(d[i].rope) || d[i].cam.mats) && d[i].n_rows > 0)
                segs.push_back({(double)(d[i].cam.mats ? tile_elems(d[i].dk) : k_image_elems(d[i].dk)),
                                i, SEG_XFORM, 0, (int64_t)d[i].B * d[i].H * cdiv(d[i].n_rows, FT_T)});
        if (!segs.empty()) {
            set_segments(M, segs);
            tile_xform_kernel<<<dim3((unsigned)seg_blocks(M)), TX_THREADS, 0, s>>>(M);
            NKV_LAUNCH_CHECK();
        }
    }
    // flash: the kernel events bracket it
    {
        std::vector<SegOrder> segs;
        for (int i = 0; i < n; ++i) {
            const FlashPlan& f = P.f[i];
            if (f.ntiles == 0 || f.splits == 0) continue;
            // eight equal runs of work items, one per XCD (see flash_block)
            segs.push_back({(double)f.ntiles / f.splits * flash_tile_cost(d[i].dk), i, SEG_FLASH, 0,
                            8 * cdiv((int64_t)d[i].B * d[i].H * f.splits * f.qtiles, 8)});
        }
        set_segments(M, segs);
    }
    const bool events = d[0].ev_begin || d[0].ev_end;
    if (seg_blocks(M) > 0) {
        const size_t smem = sizeof(FlashSmem<CK_D>);
        const bool mask = M.part[0].cur_mask != nullptr;
        rc = mask ? set_smem(flash8_kernel<true>, smem) : set_smem(flash8_kernel<false>, smem);
        if (rc) return rc;
        const dim3 grid((unsigned)seg_blocks(M));
        if (events) {
            // the dispatch itself stamps the kernel events (no marker packets
            // between the launches, which would delay the next one)
            const void* fn = mask ? (const void*)flash8_kernel<true> : (const void*)flash8_kernel<false>;
            void* args[] = {&M};
            NKV_HIP_CHECK(hipExtLaunchKernel(fn, grid, dim3(C8_THREADS), args, smem, s,
                                             (hipEvent_t)d[0].ev_begin, (hipEvent_t)d[0].ev_end, 0));
        } else if (mask) {
            flash8_kernel<true><<<grid, C8_THREADS, smem, s>>>(M);
        } else {
            flash8_kernel<false><<<grid, C8_THREADS, smem, s>>>(M);
        }
        NKV_LAUNCH_CHECK();
    } else if (events) {
        if (d[0].ev_begin) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d[0].ev_begin, s));
        if (d[0].ev_end) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d[0].ev_end, s));
    }
    const int64_t waves = 2 * (int64_t)d[0].B * d[0].H * M.part[0].qblocks;
    staged_combine_kernel<<<dim3((unsigned)cdiv(waves, CB_WAVES)), 64 * CB_WAVES, 0, s>>>(
        M, shift, sh_sb, sh_sh, ocam);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}

// Everything of a launch's ChunkParams but the workspace areas.
ChunkParams chunk_params(const ChunkLaunchDesc& d) {
    ChunkParams p;
    memset(&p, 0, sizeof(p));
    p.B = d.B;
    p.H = d.H;
    p.nch_hist = (int)chunk_count(d.n_rows);
    p.nch_total = p.nch_hist + (int)chunk_count(d.Nc);
    p.qblocks = (int)cdiv(d.Q, 32);
    // current-key chunks carry no decode: split their query blocks so that
    // the work items at the end of the grid are short (at least 16 query
    // blocks, two waves' worth, per split)
    p.cur_splits = (int)std::max<int64_t>(1, std::min<int64_t>(CK_CUR_SPLITS, p.qblocks / 16));
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
    p.q_heads = d.q_heads;
    p.q_heads_n = d.q_heads_n;
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
    p.out = d.out;
    p.o_sb = d.o_sb;
    p.o_st = d.o_st;
    p.o_sh = d.o_sh;
    p.lse = d.lse;
    p.rope = d.rope;
    p.cam = d.cam;
    p.cur_mask = d.Nc > 0 ? d.cur_mask : nullptr;
    p.q_group = d.q_group;
    p.n_groups = d.n_groups;
    p.mask_words = d.mask_words;
    return p;
}

int check_desc(const ChunkLaunchDesc& d) {
    NKV_REQUIRE(d.dk == 32 || d.dk == 64 || d.dk == 128, NKV_ERR_UNSUPPORTED,
                "key-chunk attend supports K/Q widths 32, 64 and 128");
    NKV_REQUIRE(d.B >= 1 && d.H >= 1 && d.Q >= 0 && d.n_rows >= 0 && d.Nc >= 0, NKV_ERR_INVALID,
                "bad launch shape");
    NKV_REQUIRE(d.Nc == 0 || (d.dk == CK_D && d.k_cur && d.v_cur), NKV_ERR_INVALID,
                "current keys need k_cur/v_cur and a 128-wide launch");
    // the current-key blocks index B*H*(current tiles) in 32 bits
    NKV_REQUIRE((int64_t)d.B * d.H * 2 * chunk_count(d.Nc) < ((int64_t)1 << 29), NKV_ERR_UNSUPPORTED,
                "B*H*ceil(Nc/256) must stay below 2^28");
    NKV_REQUIRE(!d.cur_mask || (d.n_groups >= 1 && d.mask_words >= cdiv(d.Nc, 32)),
                NKV_ERR_INVALID, "the current-key mask needs n_groups >= 1 and "
                "cur_mask_words >= ceil(Nc / 32)");
    NKV_REQUIRE(!d.q_heads || d.q_heads_n >= 1, NKV_ERR_INVALID, "q_heads needs q_heads_n >= 1");
    if (d.n_rows > 0) {
        int rc = check_chunk_codec(d.key);
        if (rc) return rc;
        rc = check_chunk_codec(d.value);
        if (rc) return rc;
    }
    return NKV_OK;
}

}  // namespace

size_t chunk_launch_workspace(const ChunkLaunchDesc& d) {
    if (use_staged(d)) return multi_plan(&d, 1).total;
    const int64_t nc = chunk_count(d.n_rows) + chunk_count(d.Nc);
    const size_t blocks = (size_t)d.B * d.H * nc * cdiv(d.Q, 32);
    return blocks * 32 * CK_D * sizeof(uint16_t) + blocks * 32 * 2 * sizeof(float);
}

bool staged_multi_supported(const ChunkLaunchDesc* d, int n) {
    if (n < 1 || n > NKV_MAX_PARTS) return false;
    for (int i = 0; i < n; ++i) {
        if (!use_staged(d[i]) && !(i > 0 && d[i].n_rows == 0 && d[i].Nc == 0)) return false;
        if (!staged_gemm(d[i]) || d[i].Q != d[0].Q || d[i].B != d[0].B) return false;
        if (d[i].key.r != d[0].key.r || d[i].value.r != d[0].value.r) return false;
        if (i > 0 && (d[i].Nc > 0 || d[i].cur_mask)) return false;
    }
    return d[0].dk == CK_D;
}

size_t staged_multi_workspace(const ChunkLaunchDesc* d, int n) { return multi_plan(d, n).total; }

int staged_multi_launch(hipStream_t s, const ChunkLaunchDesc* d, int n, const int32_t* const* heads,
                        const float* shift, int64_t sh_sb, int64_t sh_sh, void* workspace,
                        size_t workspace_bytes, const CameraDev& ocam) {
    NKV_REQUIRE(staged_multi_supported(d, n), NKV_ERR_UNSUPPORTED,
                "these partitions do not fit one staged launch");
    ChunkParams ps[NKV_MAX_PARTS];
    for (int i = 0; i < n; ++i) {
        int rc = check_desc(d[i]);
        if (rc) return rc;
        NKV_REQUIRE(i == 0 || (heads && heads[i]), NKV_ERR_INVALID,
                    "every partition after the first needs its head list");
        ps[i] = chunk_params(d[i]);
    }
    if (d[0].Q == 0) return NKV_OK;
    NKV_REQUIRE(d[0].q && d[0].out, NKV_ERR_INVALID, "q and out required");
    const size_t need = staged_multi_workspace(d, n);
    NKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), NKV_ERR_WORKSPACE,
                "workspace missing or smaller than the size query returned");
    return staged_run(s, d, ps, n, heads, shift, sh_sb, sh_sh, workspace, ocam);
}

int chunk_launch(hipStream_t s, const ChunkLaunchDesc& d, void* workspace, size_t workspace_bytes) {
    int rc = check_desc(d);
    if (rc) return rc;
    // the head maps of the tables are read by the decode GEMM alone
    NKV_REQUIRE((!d.key.c_heads && !d.value.c_heads) || (use_staged(d) && staged_gemm(d)),
                NKV_ERR_UNSUPPORTED, "table head maps need the staged decode GEMM");
    if (d.Q == 0) return NKV_OK;
    NKV_REQUIRE(d.q && d.out, NKV_ERR_INVALID, "q and out required");
    const size_t need = chunk_launch_workspace(d);
    NKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), NKV_ERR_WORKSPACE,
                "workspace missing or smaller than the size query returned");
    ChunkParams p = chunk_params(d);
    if (use_staged(d)) return staged_run(s, &d, &p, 1, nullptr, nullptr, 0, 0, workspace);
    const size_t qrows = (size_t)d.B * d.H * p.nch_total * p.qblocks * 32;
    p.part_o = reinterpret_cast<uint16_t*>(workspace);
    p.part_ml = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) +
                                         qrows * CK_D * sizeof(uint16_t));

    // Only reader widths 32 and 64 reach the key-chunk kernel (with ranks
    // above the resident decoder's): every call at width 128 with keys to
    // attend is staged, and current keys (the only masked
    // ones) come with width 128 alone.  A call without keys only runs the
    // combine (out = 0, lse = -inf).
    NKV_REQUIRE(d.n_rows + d.Nc == 0 || (d.dk != CK_D && d.Nc == 0), NKV_ERR_INVALID,
                "internal: a 128-wide or current-key launch reached the key-chunk kernel");
    const int64_t blocks = (int64_t)d.B * d.H * p.nch_hist;
    p.blk_base = 0;
    if (d.ev_begin) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d.ev_begin, s));
    if (blocks > 0) {
        if (d.dk == 64) launch_dk<64, false>(p, blocks, s, &rc);
        else launch_dk<32, false>(p, blocks, s, &rc);
        if (rc) return rc;
    }
    if (d.ev_end) NKV_HIP_CHECK(hipEventRecord((hipEvent_t)d.ev_end, s));
    const int64_t qblocks_total = (int64_t)d.B * d.H * p.qblocks;
    if (qblocks_total > 0) {
        chunk_combine_kernel<<<dim3((unsigned)cdiv(2 * qblocks_total, CB_WAVES)), 64 * CB_WAVES, 0,
                               s>>>(p);
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
    d.n_rows = a->hist_rows ? a->n_hist : a->N;
    d.rows = a->hist_rows;
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
    d.cur_mask = a->cur_mask;
    d.q_group = a->q_group;
    d.n_groups = a->n_groups;
    d.mask_words = a->cur_mask_words;
    return d;
}
}  // namespace

// The launch description with the call's read-time RoPE and camera (the
// workspace plan depends on the camera).
int full_desc(const nkv_attend_args* a, ChunkLaunchDesc* d) {
    *d = desc_from(a);
    if (a->camera) {
        int rc = camera_from_abi(a->camera, a->D, a->B, &d->cam);
        if (rc) return rc;
    }
    if (a->rope) {
        int rc = rope_from_abi(a->rope, a->D, &d->rope);
        if (rc) return rc;
        NKV_REQUIRE(a->N <= rope_rows_covered(a->rope),
                    NKV_ERR_INVALID, "more history tokens than the RoPE frames cover");
    }
    return NKV_OK;
}

size_t chunk_workspace_bytes(const nkv_attend_args* a) {
    ChunkLaunchDesc d;
    if (full_desc(a, &d)) return 0;
    return chunk_launch_workspace(d);
}

int chunk_check(const nkv_attend_args* a) {
    NKV_REQUIRE(a->D == CK_D, NKV_ERR_UNSUPPORTED, "key-chunk attend supports D == 128");
    NKV_REQUIRE(!a->hist_rows || (a->n_hist >= 0 && a->n_hist <= INT32_MAX), NKV_ERR_INVALID,
                "bad n_hist");
    if (a->N > 0) {
        int rc = check_segments(a->key, a->N);
        if (rc) return rc;
        rc = check_segments(a->value, a->N);
        if (rc) return rc;
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
    ChunkLaunchDesc d;
    rc = full_desc(a, &d);
    if (rc) return rc;
    return chunk_launch(s, d, workspace, workspace_bytes);
}

}  // namespace nkv

// Test hook, not part of the C ABI header: the staged planner over n <=
// NKV_MAX_PARTS partitions given as rows of nine int64 (B, H, dk, Q, n_rows,
// Nc, rK, rV, camera), then the check of every extent the staged kernels
// write against the plan (v_dk != 0 addresses the V^T images at that width,
// to show that a layout mismatch is caught).  Host arithmetic only: it runs
// without a GPU.  Returns NKV_OK, or NKV_ERR_INVALID with the violation in
// nkv_last_error; *total receives the plan's workspace bytes.
extern "C" int nkv_plan_check(const int64_t* shapes, int n, int v_dk, size_t* total) {
    using namespace nkv;
    clear_error();
    NKV_REQUIRE(shapes && n >= 1 && n <= NKV_MAX_PARTS, NKV_ERR_INVALID, "1..4 partitions");
    NKV_REQUIRE(v_dk == 0 || v_dk == 32 || v_dk == 64 || v_dk == 128, NKV_ERR_INVALID,
                "v_dk must be 0, 32, 64 or 128");
    static const float fake_mats = 0.0f;  // only its presence is read
    ChunkLaunchDesc d[NKV_MAX_PARTS];
    for (int i = 0; i < n; ++i) {
        const int64_t* r = shapes + 9 * i;
        memset(&d[i], 0, sizeof(ChunkLaunchDesc));
        d[i].B = (int)r[0];
        d[i].H = (int)r[1];
        d[i].dk = (int)r[2];
        d[i].Q = r[3];
        d[i].n_rows = r[4];
        d[i].N = r[4];
        d[i].Nc = r[5];
        d[i].key.r = (int)r[6];
        d[i].value.r = (int)r[7];
        d[i].cam.mats = r[8] ? &fake_mats : nullptr;
        NKV_REQUIRE(d[i].B >= 1 && d[i].H >= 1 && d[i].Q >= 1 && d[i].n_rows >= 0 && d[i].Nc >= 0,
                    NKV_ERR_INVALID, "bad partition shape");
        NKV_REQUIRE(use_staged(d[i]), NKV_ERR_INVALID,
                    "partition " + std::to_string(i) + " is not staged");
    }
    const MultiPlan P = multi_plan(d, n);
    if (total) *total = P.total;
    std::string why;
    NKV_REQUIRE(plan_extents_ok(P, d, n, v_dk, &why), NKV_ERR_INVALID, why);
    return NKV_OK;
}
