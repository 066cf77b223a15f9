// nkv_attend.hip -- fused INT4-codec decode + flash attention for gfx950.
//
// One 256-thread block (4 waves, one per SIMD) owns one (batch, head) pair,
// a tile of 256 queries (64 per wave) and a contiguous range of 64-token key
// tiles (a "split").  Per history tile it
//   1. streams the packed INT4 K and V coefficients with 16-byte loads and
//      unpacks them (code * scale -> bf16) into LDS,
//   2. decodes the tile on MFMA: K^T = W_K,h * Z_K^T and V = Z_V * W_V,h^T
//      (v_mfma_f32_32x32x16_bf16, fp32 accumulate), applies the reference
//      epilogue bf16(bf16(acc + bf16(mean)) + center[id]) and writes the
//      bf16 K and V^T tiles to LDS,
//   3. runs one online-softmax step: S^T = K * Q^T, P = exp2(S*c - m),
//      O^T += V^T * P^T, all on MFMA.
// Current-chunk tiles (uncompressed bf16) skip steps 1-2.  Decoded K/V only
// ever exist in LDS.  With more than one split the per-split partials
// (O, m, l) go to the caller's workspace and a combine kernel merges them.
//
// MFMA 32x32x16 bf16 operand layout (wave64): lane l supplies row (l % 32)
// of A and column (l % 32) of B with k = 8 * (l / 32) + [0, 8); accumulator
// element i of lane l is (row 8*(i/4) + 4*(l/32) + i%4, column l % 32).
// Keeping queries on the MFMA column axis (S^T, O^T) makes every softmax
// statistic lane-local except one exchange between the two half-waves.
#include "nkv_common.h"

namespace nkv {

constexpr int AT_D = 128;                     // head dim
constexpr int AT_BN = 64;                     // keys per tile
constexpr int AT_WAVES = 4;
constexpr int AT_QB = 2;                      // 32-query blocks per wave
constexpr int AT_BM = AT_WAVES * AT_QB * 32;  // 256 queries per block
constexpr int AT_RMAX = 384;
constexpr int AT_ZPAD = 8;
constexpr int AT_KPAD = 8;
constexpr int AT_VPAD = 4;

struct AttendSmem {
    uint16_t zk[AT_BN][AT_RMAX + AT_ZPAD];  // unpacked K coefficients
    uint16_t zv[AT_BN][AT_RMAX + AT_ZPAD];  // unpacked V coefficients
    uint16_t ks[AT_BN][AT_D + AT_KPAD];     // decoded K tile [token][d]
    uint16_t vt[AT_D][AT_BN + AT_VPAD];     // decoded V tile, transposed [d][token]
    int ids_k[AT_BN];
    int ids_v[AT_BN];
    float bias_k[AT_D];
    float bias_v[AT_D];
};

struct AttendParams {
    int B, H, S;          // S = splits
    int q_tiles;
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
    nkv_codec key, value;
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    float* ws_o;   // [S, B, H, Q, D]   (S > 1)
    float* ws_ml;  // [S, B, H, Q, 2]
};

__device__ __forceinline__ int read_id(const void* ids, int id_bytes, int64_t i) {
    if (id_bytes == 1) return reinterpret_cast<const uint8_t*>(ids)[i];
    if (id_bytes == 2) return reinterpret_cast<const uint16_t*>(ids)[i];
    return reinterpret_cast<const int32_t*>(ids)[i];
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

__device__ __forceinline__ bf16x8 lds_b128(const uint16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
}

// Two 8-byte LDS reads forming one bf16x8 operand: p[0..3] and p[8..11].
__device__ __forceinline__ bf16x8 lds_2x64(const uint16_t* p) {
    u32x2 a = *reinterpret_cast<const u32x2*>(p);
    u32x2 b = *reinterpret_cast<const u32x2*>(p + 8);
    u32x4 v = {a[0], a[1], b[0], b[1]};
    return as_bf16x8(v);
}

// Unpack AT_BN rows of one codec (batch-item base pointers) into LDS; rows
// >= valid become zero.  One work item = 32 codes = 16 packed bytes and one
// scale (the fused kernel requires group % 32 == 0).  Also stages center ids.
__device__ __forceinline__ void unpack_tile(uint16_t (*z)[AT_RMAX + AT_ZPAD], int* ids_s,
                                            const uint8_t* packed, const uint16_t* scales,
                                            const void* ids, const nkv_codec& c, int64_t tok0,
                                            int valid, int t) {
    const int per_row = c.r / 32;
    const int items = AT_BN * per_row;
    const int ngroups = c.r / c.group;
    for (int it = t; it < items; it += 256) {
        const int row = it / per_row;
        const int j = it - row * per_row;
        u32x4 o[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
        if (row < valid) {
            const int64_t tok = tok0 + row;
            const u32x4 w = *reinterpret_cast<const u32x4*>(packed + tok * (c.r / 2) + j * 16);
            const float s = scale_bits_to_f32(scales[tok * ngroups + (j * 32) / c.group],
                                              c.scale_dtype);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    float lo = (float)((int)((w[e] >> (8 * b)) & 15u) - 7) * s;
                    float hi = (float)((int)((w[e] >> (8 * b + 4)) & 15u) - 7) * s;
                    o[e][b] = pack_bf16x2(lo, hi);
                }
            }
        }
        u32x4* dst = reinterpret_cast<u32x4*>(&z[row][j * 32]);
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = o[e];
    }
    // ids outside the table are clamped so that a corrupt payload cannot read
    // out of bounds (valid payloads never contain them)
    if (t < AT_BN)
        ids_s[t] = (c.centers && t < valid)
                       ? min(max(read_id(ids, c.id_bytes, tok0 + t), 0), c.num_centers - 1)
                       : 0;
}

// K^T tile for d rows [32*wave, +32) and tokens [0, 64): A = W_K rows from
// global memory (16-byte loads), B = unpacked Z_K rows from LDS.  Epilogue
// writes bf16 K[token][d] (four consecutive d per 8-byte store).
__device__ __forceinline__ void decode_k(AttendSmem& sm, const nkv_codec& c,
                                         const uint16_t* centers, int HD, int h, int wave,
                                         int lane) {
    const int hf = lane >> 5, l32 = lane & 31;
    const int d0 = 32 * wave;
    const uint16_t* wrow = c.w_dec + (int64_t)(h * AT_D + d0 + l32) * c.r + 8 * hf;
    f32x16 acc0 = {}, acc1 = {};
    for (int k0 = 0; k0 < c.r; k0 += 64) {
        u32x4 wa[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) wa[u] = *reinterpret_cast<const u32x4*>(wrow + k0 + 16 * u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kk = k0 + 16 * u + 8 * hf;
            const bf16x8 b0 = lds_b128(&sm.zk[l32][kk]);
            const bf16x8 b1 = lds_b128(&sm.zk[32 + l32][kk]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(wa[u]), b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(wa[u]), b1, acc1, 0, 0, 0);
        }
    }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int tok = 32 * tb + l32;
        const uint16_t* crow = centers ? centers + (int64_t)sm.ids_k[tok] * HD + h * AT_D : nullptr;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = d0 + 8 * g + 4 * hf;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = bf16_round((tb ? acc1[4 * g + e] : acc0[4 * g + e]) + sm.bias_k[d + e]);
            if (crow) {
                const u32x2 cw = *reinterpret_cast<const u32x2*>(crow + d);
                v[0] = bf16_round(v[0] + __uint_as_float(cw[0] << 16));
                v[1] = bf16_round(v[1] + __uint_as_float(cw[0] & 0xffff0000u));
                v[2] = bf16_round(v[2] + __uint_as_float(cw[1] << 16));
                v[3] = bf16_round(v[3] + __uint_as_float(cw[1] & 0xffff0000u));
            }
            u32x2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            *reinterpret_cast<u32x2*>(&sm.ks[tok][d]) = pk;
        }
    }
}

// V tile for tokens [0, 64) and d columns [32*wave, +32): A = Z_V rows from
// LDS, B = W_V rows from global memory.  Epilogue writes bf16 V^T[d][token]
// (four consecutive tokens per 8-byte store).
__device__ __forceinline__ void decode_v(AttendSmem& sm, const nkv_codec& c,
                                         const uint16_t* centers, int HD, int h, int wave,
                                         int lane) {
    const int hf = lane >> 5, l32 = lane & 31;
    const int d = 32 * wave + l32;
    const uint16_t* wrow = c.w_dec + (int64_t)(h * AT_D + d) * c.r + 8 * hf;
    f32x16 acc0 = {}, acc1 = {};
    for (int k0 = 0; k0 < c.r; k0 += 64) {
        u32x4 wb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) wb[u] = *reinterpret_cast<const u32x4*>(wrow + k0 + 16 * u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int kk = k0 + 16 * u + 8 * hf;
            const bf16x8 a0 = lds_b128(&sm.zv[l32][kk]);
            const bf16x8 a1 = lds_b128(&sm.zv[32 + l32][kk]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, as_bf16x8(wb[u]), acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, as_bf16x8(wb[u]), acc1, 0, 0, 0);
        }
    }
    const float bias = sm.bias_v[d];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int tok = 32 * tb + 8 * g + 4 * hf;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = bf16_round((tb ? acc1[4 * g + e] : acc0[4 * g + e]) + bias);
                if (centers) {
                    const uint16_t cb =
                        centers[(int64_t)sm.ids_v[tok + e] * HD + h * AT_D + d];
                    v[e] = bf16_round(v[e] + bf16_bits_to_f32(cb));
                }
            }
            u32x2 pk = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            *reinterpret_cast<u32x2*>(&sm.vt[d][tok]) = pk;
        }
    }
}

// Copy an uncompressed current-chunk tile (rows >= valid are zero).
__device__ __forceinline__ void load_current(AttendSmem& sm, const AttendParams& p, int b,
                                             int h, int64_t tok0, int valid, int t) {
    for (int it = t; it < AT_BN * (AT_D / 8); it += 256) {
        const int row = it / (AT_D / 8);
        const int d = (it % (AT_D / 8)) * 8;
        u32x4 kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
        if (row < valid) {
            const int64_t tok = tok0 + row;
            kv = *reinterpret_cast<const u32x4*>(p.k_cur + b * p.k_sb + tok * p.k_st +
                                                 h * p.k_sh + d);
            vv = *reinterpret_cast<const u32x4*>(p.v_cur + b * p.v_sb + tok * p.v_st +
                                                 h * p.v_sh + d);
        }
        *reinterpret_cast<u32x4*>(&sm.ks[row][d]) = kv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.vt[d + 2 * e][row] = (uint16_t)(vv[e] & 0xffffu);
            sm.vt[d + 2 * e + 1][row] = (uint16_t)(vv[e] >> 16);
        }
    }
}

__global__ void __launch_bounds__(256, 1) attend_kernel(AttendParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    AttendSmem& sm = *reinterpret_cast<AttendSmem*>(smem_raw);

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
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

    // codec base pointers for batch item b
    const nkv_codec& ck = p.key;
    const nkv_codec& cv = p.value;
    const uint8_t* kpacked = ck.packed ? ck.packed + (int64_t)b * p.N * (ck.r / 2) : nullptr;
    const uint16_t* kscales = ck.scales ? ck.scales + (int64_t)b * p.N * (ck.r / ck.group) : nullptr;
    const void* kids = ck.ids ? (const void*)((const uint8_t*)ck.ids + (int64_t)b * p.N * ck.id_bytes) : nullptr;
    const uint16_t* kcent = ck.centers ? ck.centers + (int64_t)b * ck.centers_batch_stride : nullptr;
    const uint8_t* vpacked = cv.packed ? cv.packed + (int64_t)b * p.N * (cv.r / 2) : nullptr;
    const uint16_t* vscales = cv.scales ? cv.scales + (int64_t)b * p.N * (cv.r / cv.group) : nullptr;
    const void* vids = cv.ids ? (const void*)((const uint8_t*)cv.ids + (int64_t)b * p.N * cv.id_bytes) : nullptr;
    const uint16_t* vcent = cv.centers ? cv.centers + (int64_t)b * cv.centers_batch_stride : nullptr;

    if (t < AT_D) {
        sm.bias_k[t] = ck.mean ? bf16_round(ck.mean[h * AT_D + t]) : 0.0f;
        sm.bias_v[t] = cv.mean ? bf16_round(cv.mean[h * AT_D + t]) : 0.0f;
    }

    // Q^T operands: query column (l32) of block qb, d = 16*kk + 8*hf + [0, 8)
    const int64_t qbase = (int64_t)qt * AT_BM + wave * (AT_QB * 32);
    bf16x8 qr[AT_QB][AT_D / 16];
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) {
        const int64_t qi = qbase + 32 * qb + l32;
#pragma unroll
        for (int kk = 0; kk < AT_D / 16; ++kk) {
            u32x4 v = {0, 0, 0, 0};
            if (qi < p.Q)
                v = *reinterpret_cast<const u32x4*>(p.q + b * p.q_sb + qi * p.q_st + h * p.q_sh +
                                                    16 * kk + 8 * hf);
            qr[qb][kk] = as_bf16x8(v);
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

    for (int tile = tile_begin; tile < tile_end; ++tile) {
        const bool hist = tile < p.t_hist;
        const int64_t tok0 = hist ? (int64_t)tile * AT_BN : (int64_t)(tile - p.t_hist) * AT_BN;
        const int64_t len = hist ? p.N : p.Nc;
        const int valid = (int)min((int64_t)AT_BN, len - tok0);

        __syncthreads();  // previous tile fully consumed
        if (hist) {
            unpack_tile(sm.zk, sm.ids_k, kpacked, kscales, kids, ck, tok0, valid, t);
            unpack_tile(sm.zv, sm.ids_v, vpacked, vscales, vids, cv, tok0, valid, t);
            __syncthreads();
            decode_k(sm, ck, kcent, p.HD, h, wave, lane);
            decode_v(sm, cv, vcent, p.HD, h, wave, lane);
        } else {
            load_current(sm, p, b, h, tok0, valid, t);
        }
        __syncthreads();

        // ---- S^T = K * Q^T: rows = keys (32*kb + ...), cols = queries
        f32x16 s[2][AT_QB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < AT_QB; ++qb) s[kb][qb] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < AT_D / 16; ++kk) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8 a = lds_b128(&sm.ks[32 * kb + l32][16 * kk + 8 * hf]);
#pragma unroll
                for (int qb = 0; qb < AT_QB; ++qb)
                    s[kb][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qr[qb][kk], s[kb][qb],
                                                                        0, 0, 0);
            }
        }

        // ---- online softmax over the 64 keys of this tile (per query column)
        bf16x8 pb[AT_QB][4];
#pragma unroll
        for (int qb = 0; qb < AT_QB; ++qb) {
            float tmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = 32 * kb + 8 * (i / 4) + 4 * hf + (i % 4);
                    float x = s[kb][qb][i] * p.scale_log2;
                    x = key < valid ? x : -INFINITY;
                    s[kb][qb][i] = x;
                    tmax = fmaxf(tmax, x);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float m_new = fmaxf(m_run[qb], tmax);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f(m_run[qb] - m_use);
            m_run[qb] = m_new;
            float lsum = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float e = exp2f(s[kb][qb][i] - m_use);
                    s[kb][qb][i] = e;
                    lsum += e;
                }
            }
            l_run[qb] = l_run[qb] * alpha + lsum;
#pragma unroll
            for (int db = 0; db < AT_D / 32; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[qb][db][i] *= alpha;
            // P^T operands for k-steps of 16 keys: step ts uses accumulator
            // elements [8*(ts%2), +8) of key block ts/2, i.e. keys
            // 16*ts + 8*(j/4) + 4*hf + j%4 for slot j.
#pragma unroll
            for (int ts = 0; ts < 4; ++ts) {
                u32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = pack_bf16x2(s[ts / 2][qb][8 * (ts % 2) + 2 * e],
                                       s[ts / 2][qb][8 * (ts % 2) + 2 * e + 1]);
                pb[qb][ts] = as_bf16x8(v);
            }
        }

        // ---- O^T += V^T * P^T
#pragma unroll
        for (int ts = 0; ts < 4; ++ts) {
#pragma unroll
            for (int db = 0; db < AT_D / 32; ++db) {
                const bf16x8 a = lds_2x64(&sm.vt[32 * db + l32][16 * ts + 4 * hf]);
#pragma unroll
                for (int qb = 0; qb < AT_QB; ++qb)
                    o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[qb][ts], o[qb][db],
                                                                        0, 0, 0);
            }
        }
    }

    // ---- epilogue
#pragma unroll
    for (int qb = 0; qb < AT_QB; ++qb) {
        const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32);
        const int64_t qi = qbase + 32 * qb + l32;
        if (qi >= p.Q) continue;
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
// One thread per row so that lse_out may alias lse_a or lse_b.
__global__ void __launch_bounds__(256) lse_merge_kernel(int64_t rows, int D, const uint16_t* a,
                                                        int64_t as, const float* la,
                                                        const uint16_t* bb, int64_t bs,
                                                        const float* lb, uint16_t* out,
                                                        int64_t os, float* lo) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const float x = la[row], y = lb[row];
    // logaddexp: max + log1p(exp(-|x - y|)); equal inputs (including -inf) give x + ln 2
    const float l = x == y ? x + 0.69314718055994531f
                           : fmaxf(x, y) + log1pf(expf(-fabsf(x - y)));
    const float origin = isfinite(l) ? l : 0.0f;
    const float wa = expf(x - origin), wb = expf(y - origin);
    for (int d = 0; d < D; ++d) {
        const float va = bf16_bits_to_f32(a[row * as + d]);
        const float vb = bf16_bits_to_f32(bb[row * bs + d]);
        out[row * os + d] = f32_to_bf16_bits(va * wa + vb * wb);
    }
    if (lo) lo[row] = l;
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
    int q_tiles, t_hist, t_total, splits;
};

int check_attend_codec(const nkv_codec& c, int64_t N, int HD, const char* which) {
    (void)which;
    NKV_REQUIRE(c.packed && c.scales && c.w_dec, NKV_ERR_INVALID,
                "history codec needs packed, scales and w_dec");
    NKV_REQUIRE(c.r > 0 && c.r % 64 == 0, NKV_ERR_UNSUPPORTED,
                "fused attend needs r to be a multiple of 64");
    NKV_REQUIRE(c.r <= AT_RMAX, NKV_ERR_UNSUPPORTED, "fused attend supports r <= 384");
    NKV_REQUIRE(c.group > 0 && c.r % c.group == 0 && c.group % 32 == 0, NKV_ERR_UNSUPPORTED,
                "fused attend needs group to divide r and be a multiple of 32");
    NKV_REQUIRE(c.scale_dtype == NKV_DTYPE_BF16 || c.scale_dtype == NKV_DTYPE_FP16,
                NKV_ERR_INVALID, "bad scale_dtype");
    if (c.centers) {
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
    plan->q_tiles = (int)cdiv(a->Q, AT_BM);
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

}  // namespace

extern "C" size_t nkv_attend_workspace_size(const nkv_attend_args* a) {
    clear_error();
    AttendPlan pl;
    if (plan_attend(a, &pl)) return 0;
    return workspace_bytes_for(a, pl);
}

extern "C" int nkv_attend(void* stream, const nkv_attend_args* a, void* workspace,
                          size_t workspace_bytes) {
    clear_error();
    AttendPlan pl;
    int rc = plan_attend(a, &pl);
    if (rc) return rc;
    if (a->Q == 0) return NKV_OK;
    hipStream_t s = (hipStream_t)stream;
    const size_t need = workspace_bytes_for(a, pl);
    NKV_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), NKV_ERR_WORKSPACE,
                "workspace missing or smaller than nkv_attend_workspace_size()");

    AttendParams p;
    p.B = a->B;
    p.H = a->H;
    p.S = pl.splits;
    p.q_tiles = pl.q_tiles;
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
    p.key = a->key;
    p.value = a->value;
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
    static bool attr_set = false;
    if (!attr_set) {
        NKV_HIP_CHECK(hipFuncSetAttribute((const void*)attend_kernel,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
        attr_set = true;
    }
    const int64_t blocks = (int64_t)a->B * a->H * pl.q_tiles * p.S;
    attend_kernel<<<dim3((unsigned)blocks), 256, smem, s>>>(p);
    NKV_LAUNCH_CHECK();
    if (p.S > 1) {
        const int64_t threads = (int64_t)a->B * a->H * a->Q * (AT_D / 4);
        combine_kernel<<<dim3((unsigned)cdiv(threads, 256)), 256, 0, s>>>(p);
        NKV_LAUNCH_CHECK();
    }
    return NKV_OK;
}

extern "C" int nkv_lse_merge(void* stream, int64_t rows, int D, const uint16_t* a,
                             int64_t a_stride, const float* lse_a, const uint16_t* b,
                             int64_t b_stride, const float* lse_b, uint16_t* out,
                             int64_t out_stride, float* lse_out) {
    clear_error();
    NKV_REQUIRE(rows >= 0 && D > 0, NKV_ERR_INVALID, "rows must be >= 0 and D > 0");
    if (rows == 0) return NKV_OK;
    NKV_REQUIRE(a && b && lse_a && lse_b && out, NKV_ERR_INVALID, "null pointer");
    lse_merge_kernel<<<dim3((unsigned)cdiv(rows, 256)), 256, 0, (hipStream_t)stream>>>(
        rows, D, a, a_stride, lse_a, b, b_stride, lse_b, out, out_stride, lse_out);
    NKV_LAUNCH_CHECK();
    return NKV_OK;
}
