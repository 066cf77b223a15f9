/*
 * nanokv.h -- C ABI of libnanokv_hip.so, the MI355X (gfx950) implementation
 * of NanoKV's codec-native historical attention.
 *
 * Conventions (all entry points):
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Work is enqueued asynchronously; the library never synchronises.
 *  - Every pointer is device memory owned and allocated by the caller.  The
 *    library allocates no device memory; kernels that need scratch take a
 *    caller-provided workspace whose size is queried first.
 *  - Return 0 (NKV_OK) or a negative NKV_ERR_* code.  The message for the
 *    last failure on the calling thread is returned by nkv_last_error().
 *  - bf16 and fp16 values travel as uint16_t bit patterns.
 *  - Shapes are validated on the host before any launch; invalid shapes are
 *    rejected with NKV_ERR_INVALID and launch nothing.
 *
 * Reference interfaces replaced (paths relative to the NanoKV tree;
 * MG = models/Matrix-Game-3.5/fast/diffsynth/models/nanokv_codec.py,
 * CN = models/Matrix-Game-3.5/fast/codec_native):
 *  nkv_quant_pack  <- MG:349-351 + _pack_int4 MG:282-292; HY Triton
 *                     int4_quant_pack_per_row (kv_codec_triton.py:60-81)
 *  nkv_unpack      <- unpack_int4_scaled (nanokv_codec_kernels.py:30-61),
 *                     latent_kernel.read (CN/latent_kernel.py:18-23)
 *  nkv_assign      <- the argmin step of semantic_residual MG:315-321;
 *                     HY _joint_euclid_assign_kernel (kv_codec_triton.py:238-273)
 *  nkv_encode      <- encode_tensor MG:333-365 with given shared centers
 *  nkv_c64_fit     <- the C64 center fit of semantic_residual MG:301-330
 *  nkv_decode      <- _decode_method_segments MG:393-455, decode_tensor
 *                     MG:368-390, decode_pair_selected MG:801-861
 *  nkv_attend      <- decode_pair_values (MG:542) followed by the history
 *                     attention of causal_self_attention_kv
 *                     (wan_video_dit.py:488-627) / attention_lse
 *                     (CN/core.py:45-72), fused into one kernel
 *  nkv_lse_merge   <- merge (CN/core.py:33-42), fast_kernels._merge
 *                     (CN/fast_kernels.py:30-54)
 *  nkv_lift_lse_combine <- HY lift_lse_combine (HYP:1807-1867; kernels
 *                     _main_lift_lse_combine_kernel / _prope_lift_lse_combine_kernel
 *                     HYP:883-1014), HYP = models/HY-WorldPlay/fast/hyvideo/models/
 *                     transformers/modules/codec_native_position_triton.py
 *  nkv_finish      <- LingBot finish (LBF:36-46, kernel _finish LBF:10-34),
 *                     LBF = models/LingBot-World-2.0/fast/wan/modules/
 *                     codec_native_finish_triton.py
 *  nkv_fast_attend <- hybrid_attention (CN/core.py:278-310) and the partition
 *                     reads of maybe_attention (CN/mg35.py:100-357)
 *  nkv_int8_pack   <- _pack_operator MG:108-131 (INT8 operator storage)
 *  nkv_int8_dequant <- unpack_int8_weight (nanokv_codec_kernels.py:64-82),
 *                     the INT8 branch of _operator_linear MG:145-152
 *  nkv_camera_apply, nkv_attend_args.camera <- the camera PRoPE transforms of
 *                     prope_attention_by_frame_indices (wan_video_dit.py:85-128)
 *                     and the fused camera kernel (CN/camera_kernel.py:8-36)
 *  nkv_rope_apply  <- rope_apply (wan_video_dit.py:185-192) with the 3-D
 *                     frequencies of _kv_freqs (pipelines/wan_video.py:3322-3341);
 *                     nkv_attend_args.rope fuses the same rotation into the
 *                     decode (the read-time RoPE of cached keys,
 *                     wan_video_dit.py:538-546)
 */
#ifndef NANOKV_H
#define NANOKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKV_ABI_VERSION 7

enum nkv_status {
    NKV_OK = 0,
    NKV_ERR_INVALID = -1,     /* bad shape, pointer or parameter */
    NKV_ERR_UNSUPPORTED = -2, /* valid request this build does not implement */
    NKV_ERR_HIP = -3,         /* a HIP runtime call failed */
    NKV_ERR_WORKSPACE = -4    /* workspace missing or too small */
};

enum nkv_scale_dtype { NKV_DTYPE_BF16 = 0, NKV_DTYPE_FP16 = 1 };

/* Work decomposition of nkv_attend.  Both give the same attention (within
 * bf16 rounding of the partials); they differ in cost:
 *  QUERY_TILES  a block owns a 256-query tile and a range of 32-key tiles and
 *               decodes each tile into registers and LDS right before
 *               attending it (decoded K/V never leave the CU), so every
 *               history tile is decoded once per query tile; partials only
 *               across the `splits` key ranges.
 *  KEY_CHUNKS   every history tile is decoded once per head (the staged
 *               schedule): one launch decodes each 128-key tile into the
 *               call's workspace in the attention kernel's LDS layout (K and
 *               V^T images, 64 KiB per tile: 176 MB at 24 heads x 12,480
 *               keys), a flash launch streams the tiles through LDS with each
 *               query block's O in registers over a key split, and a combine
 *               merges the splits' bf16 partials by LSE.
 *  AUTO         KEY_CHUNKS whenever the codecs fit it (D = 128, ranks that
 *               are multiples of 64, scale groups that are multiples of 32),
 *               QUERY_TILES otherwise. */
enum nkv_schedule {
    NKV_SCHEDULE_AUTO = 0,
    NKV_SCHEDULE_QUERY_TILES = 1,
    NKV_SCHEDULE_KEY_CHUNKS = 2
};

/* Arithmetic of the quantiser (see nkv_quant_pack). */
enum nkv_quant_mode { NKV_QUANT_FP32 = 0, NKV_QUANT_BF16 = 1 };

/* ABI version of the loaded library (NKV_ABI_VERSION at build time). */
int nkv_abi_version(void);

/*
 * INT8 codec operators (the mg35_worldplay_operator_int8_v1 storage).
 * nkv_int8_pack (_pack_operator, MG:108-131): w [rows, cols] fp32 in groups
 * of `group` columns; per (row, group) s = max(amax|w|, 1e-12) / 127 (fp32),
 * q = clamp(rint(w / s), -127, 127), scale[row, g] = bf16(s).
 * nkv_int8_dequant (unpack_int8_weight, nanokv_codec_kernels.py:64-82):
 * out [rows, cols] = bf16(q * scale[row, col / group]).
 */
int nkv_int8_pack(void* stream, const float* w, int64_t rows, int cols, int group, int8_t* q,
                  uint16_t* scale);
int nkv_int8_dequant(void* stream, const int8_t* q, const uint16_t* scale, int64_t rows, int cols,
                     int group, uint16_t* out);

/*
 * Rotary position embedding of cached keys, applied at read time
 * (rope_apply, wan_video_dit.py:185-192, over the per-token frequencies
 * that _kv_freqs builds from precompute_freqs_cis_3d, wan_video_dit.py:168-182).
 * The positions follow the codec row n of a key: frame f = n / (grid_h*grid_w)
 * at temporal position frame_pos[f], row (n % (grid_h*grid_w)) / grid_w and
 * column n % grid_w.  Complex pair p (dims 2p, 2p+1) of a head rotates by
 *   p < pt            cs_t[frame_pos[f]][p]
 *   pt <= p < pt+ph   cs_h[row][p - pt]
 *   otherwise         cs_w[col][p - pt - ph]
 * where every entry is an fp64 (cos, sin) pair (the reference's complex128
 * polar(1, angle) tables; a (1, 0) band is no rotation, as the reference's
 * prope_disable_t_rope).  In fp64 with each product rounded:
 *   y[2p] = x[2p] c - x[2p+1] s,  y[2p+1] = x[2p] s + x[2p+1] c,
 * rounded to fp32 and then to bf16 (torch's float64 -> bfloat16).
 * pt + ph + pw must be D / 2.  Table pointers are device memory.
 * Per-row table (cs_rows != NULL, the reference's own per-token cache_freqs
 * layout [n, 1, D/2] complex128 viewed as real): pair p of row n rotates by
 * cs_rows[n][p] (n clamped to [0, n_rows)); the bands, frame_pos and the
 * grid are then ignored.
 */
typedef struct nkv_rope {
    const double* cs_t;           /* [n_t, pt, 2] temporal band */
    const double* cs_h;           /* [grid_h, ph, 2] row band */
    const double* cs_w;           /* [grid_w, pw, 2] column band */
    const int32_t* frame_pos;     /* [n_frames] cs_t row of each frame */
    int64_t n_frames;
    int n_t;
    int pt, ph, pw;
    int grid_h, grid_w;
    int _pad;
    const double* cs_rows;        /* [n_rows, D/2, 2] per-row table, or NULL */
    int64_t n_rows;
} nkv_rope;

/*
 * Camera PRoPE (prope_attention_by_frame_indices, wan_video_dit.py:85-128;
 * layouts of prope_attention.py:9-24, 120-176): each frame of rows has a set
 * of four sub-frame 4x4 matrices (P^-1 for keys and values, P^T for queries,
 * P for outputs); 4-vectors of each head are multiplied by their sub-frame's
 * matrix, y = M x, with the matrix entries rounded to bf16, the products
 * summed exactly, and the result rounded fp32 -> bf16 (camera_kernel.py:8-36,
 * fp64 accumulation).  Layouts: FULL tiles all D dims (D % 64 == 0): dim
 * d = ((p*4 + c)*4 + j)*(D/64) + r, vector over j, sub-frame c; SF13 puts
 * sub-frame 1 on dims [0, 16) and 3 on [16, 32) as contiguous 4-vectors and
 * leaves the rest.  Row n of batch item b uses matrix set
 * frame_mat[n / tokens_per_frame] of mats + b * mats_bs (frame and set
 * indices clamped to range).  mats must be 16-byte aligned and mats_bs a
 * multiple of 4.  n_batches is the number of matrix batches mats holds; a
 * call over B batch items needs mats_bs == 0 (one set shared by every item)
 * or B <= n_batches.
 */
enum nkv_camera_layout { NKV_CAMERA_FULL = 0, NKV_CAMERA_SF13 = 1 };

typedef struct nkv_camera {
    const float* mats;            /* [batches, n_mats, 4, 4, 4] fp32, device */
    int64_t mats_bs;              /* floats between batch items (0: shared) */
    int n_mats;
    int layout;                   /* nkv_camera_layout */
    const int32_t* frame_mat;     /* [n_frames] matrix set of each frame, device */
    int64_t n_frames;
    int tokens_per_frame;
    int n_batches;                /* matrix batches in mats (>= B unless mats_bs == 0) */
} nkv_camera;

/* out[b, s, h, :] = the camera transform of x[b, s, h, :] at row rows[s]
 * (rows NULL: row s); layout as nkv_rope_apply.  out may be x. */
int nkv_camera_apply(void* stream, const nkv_camera* camera, int B, int64_t S, int H, int D,
                     const uint16_t* x, int64_t x_sb, int64_t x_st, int64_t x_sh,
                     const int32_t* rows, uint16_t* out, int64_t o_sb, int64_t o_st,
                     int64_t o_sh);

/*
 * out[b, s, h, :] = RoPE of x[b, s, h, :] at the position of row rows[s]
 * (rows NULL: row s), x and out [B, S, H, D] bf16 addressed as
 * x[b*x_sb + s*x_st + h*x_sh + d] (out likewise; out may be x).  D even.
 */
int nkv_rope_apply(void* stream, const nkv_rope* rope, int B, int64_t S, int H, int D,
                   const uint16_t* x, int64_t x_sb, int64_t x_st, int64_t x_sh,
                   const int32_t* rows, uint16_t* out, int64_t o_sb, int64_t o_st,
                   int64_t o_sh);

/* Message of the last failed call on this thread ("" if none). */
const char* nkv_last_error(void);

/*
 * INT4 symmetric quantisation of fp32 coefficients, packed two per byte.
 *   coeff  [rows, r] fp32        packed [rows, r/2] uint8
 *   scales [rows, r/group] bf16 or fp16 bits (scale_dtype)
 * Per (row, group): s = max(amax|x|, FLT_EPSILON) / 7 (IEEE division);
 * code = clamp(round_half_even(x / s), -7, 7); byte j of a row holds codes
 * 2j (low nibble) and 2j+1 (high nibble) as code + 7; scales store cast(s).
 * quant_mode NKV_QUANT_BF16 reproduces MG's bf16 tensor arithmetic: the
 * input, amax, s and x/s are each rounded to bf16 (MG:138-153, 349-351).
 * group must divide r; r must be even.  group == r is the reference's
 * one-scale-per-row layout.
 */
int nkv_quant_pack(void* stream, const float* coeff, int64_t rows, int r, int group,
                   int scale_dtype, int quant_mode, uint8_t* packed, uint16_t* scales);

/*
 * Unpack INT4 codes and apply their group scale:
 *   latent[i, j] = bf16( float(code[src, j]) * float(scale[src, j / group]) )
 * with src = row_index ? row_index[i] : i.  latent is [rows, r] bf16 bits.
 */
int nkv_unpack(void* stream, const uint8_t* packed, const uint16_t* scales, int scale_dtype,
               const int32_t* row_index, int64_t rows, int r, int group, uint16_t* latent);

/*
 * Nearest-center assignment: ids[n] = argmin_c ||x_n - c||^2 over the bf16
 * table (first index on ties), decided in fp64 from the fp32/bf16 inputs.
 *   x [rows, HD] fp32, centers [C, HD] bf16, ids [rows] of id_bytes
 *   (1 = uint8 for C <= 256, 2 = uint16 for C <= 65536, 4 = int32).
 */
int nkv_assign(void* stream, const float* x, const uint16_t* centers, int64_t rows, int C,
               int HD, void* ids, int id_bytes);

/*
 * One immutable segment of a codec cache (a payload of the reference's
 * worldplay_segments_v1 list, nanokv_codec.py:600-609): its own packed
 * codes, scales, center ids and center table.  Segment s holds codec rows
 * [row_start, row_start + rows); the segments of a codec are in row order and
 * contiguous from row 0 (row_start of segment s = the sum of the rows before
 * it).  center_base = the sum of num_centers of the segments before it (the
 * row of this segment's table in the concatenation of all tables, used when
 * the library projects the tables of every segment at once).  Every segment
 * of a codec has centers, or none does.
 */
typedef struct nkv_segment {
    const uint8_t* packed;        /* [B, rows, r/2] */
    const uint16_t* scales;       /* [B, rows, r/group] */
    const void* ids;              /* [B, rows] of id_bytes, or NULL (no centers) */
    const uint16_t* centers;      /* [B or 1, num_centers, HD] bf16, or NULL */
    int64_t row_start;
    int64_t rows;
    int64_t centers_batch_stride; /* elements between batch tables; 0 = shared */
    int64_t center_base;
    int num_centers;
    int id_bytes;
} nkv_segment;

/* One K or V codec as stored in the cache: either one flat array of all rows
 * (packed, scales, ids, centers below) or, with n_segments > 0, the segment
 * table (the reference's segment list, decoded segment by segment with each
 * segment's own center table, nanokv_codec.py:393-455), given twice: as a host
 * array the library validates and plans from, and as the same table in device
 * memory that the kernels read.  With segments, packed/scales/ids/centers,
 * id_bytes, num_centers and centers_batch_stride of the codec are ignored;
 * r, group, scale_dtype, w_dec and mean apply to every segment. */
typedef struct nkv_codec {
    const uint8_t* packed;        /* [B, N, r/2] */
    const uint16_t* scales;       /* [B, N, r/group] */
    const void* ids;              /* [B, N] of id_bytes, or NULL when centers == NULL */
    const uint16_t* centers;      /* [B or 1, C, HD] bf16, or NULL (no center add) */
    const uint16_t* w_dec;        /* [HD, r] bf16 decoder weight (F.linear layout) */
    const float* mean;            /* [HD] fp32 bias (applied as bf16), or NULL */
    int r;
    int group;
    int scale_dtype;
    int id_bytes;
    int num_centers;
    int n_segments;               /* 0: the flat arrays above */
    int64_t centers_batch_stride; /* elements between batch tables; 0 = shared */
    const nkv_segment* segments;      /* host array of n_segments */
    const nkv_segment* segments_dev;  /* the same table in device memory */
} nkv_codec;

/*
 * Encode a chunk with given shared centers (assign -> residual -> encoder
 * projection -> quantise/pack), following encode_tensor MG:333-365:
 *   residual = x - fp32(center[id]) - mean, cast to bf16 (MG:326-330, 346)
 *   coeff    = residual @ w_enc^T, fp32 accumulate (MG:134-153)
 *   packed, scales = nkv_quant_pack(coeff)
 * `coeff` is an output the caller allocates ([rows, r] fp32); it is also the
 * exact input the quantiser saw.  With centers == NULL no center is
 * subtracted and ids is not written (the reference's pca rung).
 */
typedef struct nkv_encode_args {
    int64_t rows;                 /* tokens in this batch item */
    int HD;
    int r;
    int group;
    int scale_dtype;
    int quant_mode;
    int num_centers;
    int id_bytes;
    int ids_in;                   /* 1: ids hold each row's center on input (no search) */
    const float* x;               /* [rows, HD] fp32 */
    const uint16_t* centers;      /* [C, HD] bf16 or NULL */
    const float* mean;            /* [HD] fp32 or NULL */
    const uint16_t* w_enc;        /* [r, HD] bf16 */
    void* ids;                    /* out [rows] */
    float* coeff;                 /* out [rows, r] fp32 */
    uint8_t* packed;              /* out [rows, r/2] */
    uint16_t* scales;             /* out [rows, r/group] */
    /* bf16 rows in place of x (read as the reference's value.float(), which
     * is exact), or NULL; needs HD % 256 == 0 and 16-byte aligned rows,
     * and to search, at most 256 centers and HD <= 16384. */
    const uint16_t* x_bf16;
    int64_t x_stride;             /* elements between rows of x / x_bf16; 0 = HD */
} nkv_encode_args;

int nkv_encode(void* stream, const nkv_encode_args* args);

/*
 * n (1..8) independent encodes of one shape in one launch per stage (the
 * K and V of a layer, batch items): every problem has its own rows, inputs,
 * operator, centers, mean and outputs, and all share HD, r, group,
 * scale_dtype, quant_mode, the center count and id type, ids_in, the input
 * dtype and whether a mean is given.  Each problem's results are those of
 * nkv_encode on it.  No counterpart in the reference (encode_tensor, MG:
 * 333-365, encodes one tensor per call).
 */
int nkv_encode_batch(void* stream, const nkv_encode_args* args, int n);

/*
 * Per-chunk C64 center fit (semantic_residual, MG:301-330), per batch item:
 * the centers start as the rows init_rows[0 .. C) (the reference draws them
 * with randperm(S, Generator(cpu).manual_seed(20260804 + layer))[:C]); each
 * of `iterations` rounds labels every row with its nearest center (exact
 * fp64 decision, first index on ties, as nkv_assign) and replaces every
 * center that has rows by their mean, fp32(fp64 sum in row order) / count in
 * fp32 (the reference sums in fp32 in library order); a center without rows
 * keeps its value.  labels are the last round's (zero for 0 rounds).
 *   x [B, S, HD] fp32; centers out [B, C, HD] fp32; labels out [B, S] int32;
 *   1 <= C <= min(S, 256).
 */
size_t nkv_c64_fit_workspace_size(int B, int64_t S, int C);
int nkv_c64_fit(void* stream, const float* x, int B, int64_t S, int HD, int C, int iterations,
                const int32_t* init_rows, float* centers, int32_t* labels, void* workspace,
                size_t workspace_bytes);

/*
 * Full-width decode of all or selected rows to bf16 (the reference's decode
 * path, used for decode_value / decode_pair_selected):
 *   rows = bf16(latent @ w_dec^T + bf16(mean))                  MG:438-443
 *   rows = bf16(float(rows) + float(center[id]))                MG:445-454
 * out [B, rows, HD] bf16.  row_index (NULL = all N) selects rows of every
 * batch item.  The codec must be flat (n_segments == 0): each segment of a
 * segment list is decoded by its own call, as the reference decodes them.
 */
typedef struct nkv_decode_args {
    int B;
    int HD;
    int64_t N;                    /* tokens per batch item in the codec */
    int64_t rows;                 /* output rows per batch item */
    const int32_t* row_index;     /* [rows] or NULL (rows == N) */
    nkv_codec codec;
    uint16_t* out;
} nkv_decode_args;

int nkv_decode(void* stream, const nkv_decode_args* args);

/*
 * Decode-and-attend in one call: softmax(q k^T * softmax_scale) v over the
 * keys [decoded history (N tokens); current chunk (Nc tokens)], non-causal.
 * History K/V rows are decoded tile by tile with the nkv_decode arithmetic:
 * once per head into the workspace, in the attention kernel's LDS layout
 * (KEY_CHUNKS, the staged schedule), or once per 256-query tile into
 * registers and LDS right before they are attended (QUERY_TILES); no
 * decoded K/V tensor is produced.
 *   q       [B, Q, H, D] addressed as q[b*q_sb + t*q_st + h*q_sh + d]
 *   k_cur   [B, Nc, H, D] (k_sb/k_st/k_sh), v_cur likewise (v_*)
 *   out     [B, Q, H, D] bf16 (o_sb/o_st/o_sh)
 *   lse     [B, H, Q] fp32 natural-log row log-sum-exp, or NULL
 * q, out, k_cur and v_cur are read and written as 16-byte pieces: they must be
 * 16-byte aligned with strides divisible by 8 (NKV_ERR_INVALID otherwise).
 * key/value codecs decode to HD = H * D columns; head h reads columns
 * [h*D, (h+1)*D).  An empty key set gives out = 0 and lse = -inf
 * (attention_lse, CN/core.py:48-49).  D = 128, or D < 128 with D % 8 == 0:
 * narrower heads (BASELINE config 0 has D = 64) run the D = 128 kernels on
 * operands padded with zero columns inside the workspace (exact: the zero
 * columns add nothing to q.k and give zero output columns), without RoPE,
 * the camera or segmented codecs.
 * rope (host pointer, NULL = none): history keys are rotated after decode at
 * the positions of their codec rows (see nkv_rope); q and k_cur are taken as
 * already rotated.  RoPE runs on the KEY_CHUNKS schedule (AUTO picks it).
 * camera (host pointer, NULL = none): history keys (after RoPE) and values are
 * multiplied by their frame's P^-1 after decode (see nkv_camera); q, k_cur and
 * v_cur are taken as already transformed and the caller applies P to out.
 * The camera also runs on the KEY_CHUNKS schedule.
 * hist_rows (device, NULL = rows 0 .. N-1 in order): the codec rows attended,
 * n_hist of them (rows outside [0, N) are clamped; an empty list is a
 * non-NULL pointer with n_hist = 0); the reference's frame selection by
 * cache chunk id (wan_video_dit.py:509-530).
 * cur_mask (device, NULL = every current key visible): visibility bits of the
 * current keys per query group, bit k % 32 of word cur_mask[g*cur_mask_words
 * + k/32] for current key k seen by the queries of group g; q_group[t] (device,
 * NULL = group 0) is the group of query t (groups clamped to [0, n_groups)).
 * Query groups with identical visibility are attention_grouped_mask's
 * (CN/core.py:94-103); the bits carry any boolean mask of attention_lse
 * (CN/core.py:45-72) and the hook's hole/chunk-id keep masks
 * (CN/mg35.py:258-283).  A query that sees no key gets out = 0, lse = -inf.
 * rope, camera, hist_rows, cur_mask and codec segments run on the
 * KEY_CHUNKS schedule (AUTO picks it when any is given).
 */
typedef struct nkv_attend_args {
    int B;
    int H;
    int D;
    int splits;                   /* QUERY_TILES key splits; 0 = choose automatically */
    int64_t Q;
    int64_t N;
    int64_t Nc;
    float softmax_scale;
    int schedule;                 /* NKV_SCHEDULE_*: work decomposition */
    const uint16_t* q;
    int64_t q_sb, q_st, q_sh;
    const uint16_t* k_cur;
    int64_t k_sb, k_st, k_sh;
    const uint16_t* v_cur;
    int64_t v_sb, v_st, v_sh;
    nkv_codec key;
    nkv_codec value;
    uint16_t* out;
    int64_t o_sb, o_st, o_sh;
    float* lse;
    /* Optional instrumentation: hipEvent_t handles (as void*) recorded on
     * `stream` immediately before and after the main attention kernel (the
     * fused kernel; with the staged schedule, the flash kernel after the
     * history decode; never the split-combine), for per-kernel timing.
     * NULL = not recorded. */
    void* ev_kernel_begin;
    void* ev_kernel_end;
    const nkv_rope* rope;
    const nkv_camera* camera;
    const int32_t* hist_rows;     /* [n_hist] codec rows attended, or NULL (all N) */
    int64_t n_hist;
    const uint32_t* cur_mask;     /* [n_groups, cur_mask_words] or NULL */
    const int32_t* q_group;       /* [Q] mask group of each query, or NULL */
    int n_groups;
    int cur_mask_words;           /* >= ceil(Nc / 32) */
} nkv_attend_args;

/* Bytes of workspace nkv_attend needs for these arguments (0 if none). */
size_t nkv_attend_workspace_size(const nkv_attend_args* args);

int nkv_attend(void* stream, const nkv_attend_args* args, void* workspace,
               size_t workspace_bytes);

/*
 * Allocation-free nkv_attend.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory or pass a workspace (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, arithmetic and results as nkv_attend, but the scratch is a
 * static array of NKV_STATIC_SCRATCH_BYTES per GPU inside the library (held
 * until the process ends); a call that needs more (nkv_attend_workspace_size)
 * fails with NKV_ERR_WORKSPACE and launches nothing.  No part of the scratch
 * needs to start at zero: every byte a call reads it wrote first (the
 * flash kernel copies no tile the decode left unwritten).  Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams, two threads) race; serialise them.  The stream must belong to the
 * current device.  Allocates nothing (no hipMalloc, no allocating library
 * routine).
 */
#define NKV_STATIC_SCRATCH_BYTES (64u << 20)
int nkv_attend_static(void* stream, const nkv_attend_args* args);

/*
 * One reader group of NanoKV-Fast (ReaderGroup, CN/core.py:155-204): its
 * heads read the low (unprotected) history rows through learned projections
 *   q_low = bf16(q_h . q_reduce[i])                         [Q, d]
 *   k_low = bf16(bf16(latent_K . k_read[i]^T + kbias[i]) + kcent[i][id])
 *   v_low = bf16(bf16(latent_V . v_read[i]^T + vbias[i]) + vcent[i][id])
 * with kcent[i] = bf16(center columns of head h . k_affine[i]) and
 * kbias[i] = bf16(bf16(mean_h) . k_affine[i]) (V likewise with v_affine);
 * latent = the unpacked INT4 codes (nkv_unpack).  A NULL q_reduce / k_affine
 * / v_affine is the identity (the reference's identity flags).  The value
 * width and the lift are D (identity lift).  All pointers are device memory.
 */
typedef struct nkv_reader_group {
    int num_heads;
    int d;                        /* K/Q reader width: 32, 64 or 128 (== D for identity) */
    const int32_t* heads;         /* [num_heads] layer head indices */
    const uint16_t* q_reduce;     /* [num_heads, D, d] bf16 or NULL */
    const uint16_t* k_read;       /* [num_heads, d, rK] bf16 */
    const uint16_t* v_read;       /* [num_heads, D, rV] bf16 */
    const uint16_t* k_affine;     /* [num_heads, D, d] bf16 or NULL */
    const uint16_t* v_affine;     /* [num_heads, D, D] bf16 or NULL */
    /* RoPE of the reader keys and queries (rope_selected, CN/core.py:75-91):
     * [num_heads, d/2] int32, the original pair (indices[:, 0::2] / 2) of each
     * pair of the d-wide key/query; NULL = pair j (d == D).  Used only when
     * the call applies RoPE. */
    const int32_t* rope_pairs;
    /* Camera of the reader keys and queries (camera_selected, CN/core.py:
     * 110-137): [num_heads, d/8] int32, the camera sub-frame of each 8-dim
     * block of the d-wide key/query (the original block's (indices[8j] / 8) % 4);
     * NULL = block j uses sub-frame j % 4 (d == D).  Within a block the two
     * 4-vectors are dims {0, 2, 4, 6} and {1, 3, 5, 7}, as in the full
     * layout.  Used only when the call applies a camera. */
    const int32_t* cam_blocks;
} nkv_reader_group;

/*
 * NanoKV-Fast mixed-dimensional history attention (hybrid_attention
 * CN/core.py:278-310 with maybe_attention's partitions CN/mg35.py:192-348):
 *   native partition: every head attends to the history rows protect_rows
 *     (decoded at full width, as nkv_attend) and the current keys;
 *   low partition: the heads of each reader group attend to the history
 *     rows low_rows through the group's readers;
 *   out = merge of the two by log-sum-exp (CN/core.py:33-42), per head.
 * attend carries q, the current K/V, the key/value codecs (decoders for the
 * native partition), out and lse, as for nkv_attend (its N is the codec's
 * token count; splits and schedule are ignored).  Every head should belong
 * to exactly one group (CN/core.py:213-215); a head in no group keeps the
 * native partition alone.  A head listed by more than one group is invalid
 * (the reference rejects such groups, CN/core.py:213-215); the heads arrays
 * are device memory, so the call cannot check it, and such a head's output is
 * unspecified (one staged launch merges the first group listing it, the
 * per-group path every one in turn).  The Python layer (ReaderLayer) refuses
 * such groups before any call.  Returns NKV_ERR_UNSUPPORTED for D != 128.
 * RoPE (attend.rope != NULL, CN/mg35.py:207-214, 305-336): the native
 * partition's history keys are rotated at their codec rows and attend.q is
 * taken as already rotated; each reader group forms its queries from the
 * pre-RoPE queries q_pre, q_low = bf16(q_pre . q_reduce), and rotates the
 * pairs rope_pairs of q_low at the query positions q_rope (query t at row t)
 * and of k_low at the codec rows' positions (attend.rope).
 * Camera (attend.camera != NULL, the FULL layout, CN/mg35.py:253-257,
 * 310-346): attend.camera holds P^-1 of the history rows; the native
 * partition's history keys and values are transformed in-kernel and attend.q,
 * k_cur and v_cur are taken as already transformed; each reader group's q_low
 * is transformed by P^T of the query rows (q_camera, query t at row t) and
 * k_low / v_low by P^-1 on their blocks (cam_blocks).  P of the query rows
 * goes on out after the merge: by the call when o_camera is given, else by
 * the caller (as for nkv_attend).  With a value lift folded into the value
 * reader (block-selection or identity lifts) P commutes with the lift, and
 * it commutes with the merge (one P per query row for both partitions); the
 * reference applies it to each partition's bf16 output before the merge
 * (CN/mg35.py:310-347), so only the bf16 rounding points differ.
 * Value-mean correction (low_shift != NULL; LingBot codec_native_attention.py
 * :779-785 and finish, codec_native_finish_triton.py:31-32): low_shift[b, h]
 * ([B, H, D] fp32, strides ls_sb, ls_sh, unit d stride) is added to every
 * low-partition value of head h, i.e. to the low output before the merge;
 * the reference's mean - projected, where the lift is low-rank.
 */
typedef struct nkv_fast_args {
    nkv_attend_args attend;
    const int32_t* protect_rows;  /* [n_protect] codec rows, device memory */
    int64_t n_protect;
    const int32_t* low_rows;      /* [n_low] codec rows, device memory */
    int64_t n_low;
    int num_groups;
    int _pad;
    const nkv_reader_group* groups;  /* host array of num_groups */
    const uint16_t* q_pre;        /* [B, Q, H, D] bf16 pre-RoPE queries (with RoPE) */
    int64_t qp_sb, qp_st, qp_sh;
    const nkv_rope* q_rope;       /* query positions (with RoPE), host pointer */
    const nkv_camera* q_camera;   /* P^T of the query rows (with a camera), host pointer */
    const float* low_shift;       /* [B, H, D] fp32 low value shift, or NULL */
    int64_t ls_sb, ls_sh;
    /* P of the query rows, applied to out (FULL layout) once the partitions
     * are merged: out = bf16(P . out) as nkv_camera_apply computes it, the
     * caller's last step of the camera attention (CN/mg35.py:310-347).
     * Host pointer, or NULL: out is left in the values' frame. */
    const nkv_camera* o_camera;
} nkv_fast_args;

/* Bytes of workspace nkv_fast_attend needs for these arguments. */
size_t nkv_fast_attend_workspace_size(const nkv_fast_args* args);

int nkv_fast_attend(void* stream, const nkv_fast_args* args, void* workspace,
                    size_t workspace_bytes);

/*
 * Rows of a [B, S, H, D] bf16 tensor read through a reader group, for MG's
 * low_native extension (mg35.py:241-249, 324-336): the mosaic / current
 * tokens moved into the low partition, keys and values projected from their
 * pre-RoPE rows by the group's affine (einsum('bhnd,hde->bhne'), bf16), and
 * the group query.  For head i of the group (original head heads[i]):
 *   y = bf16(x[b, s, heads[i], :] . w[i])          w [nh, D, E] bf16 (NULL:
 *                                                  the identity, E = D)
 *   y rotated on its pairs at the position of row s (rope, NULL = none;
 *   pairs [nh, E/2]: original pair of reader pair j, NULL = pair j), the
 *   arithmetic of nkv_rope_apply (rope_selected, CN/core.py:75-91)
 *   y multiplied on its 8-dim blocks by the camera of row s (camera, FULL
 *   layout, NULL = none; blocks [nh, E/8]: sub-frame of reader block j,
 *   NULL = j % 4), the arithmetic of the reader queries of nkv_fast_attend
 *   (camera_selected, CN/core.py:110-137)
 * out [B, S, nh, out_width] bf16 (contiguous), columns E .. out_width - 1
 * zero, so that a reader key or query of width E < 128 can be attended by
 * nkv_attend at width 128 (the zero columns add nothing to q.k).  E and
 * out_width are multiples of 8, E <= out_width, D <= 512.  No counterpart
 * as one function in the reference.
 */
typedef struct nkv_reader_rows_args {
    int B, H, D, E, nh, out_width;
    int64_t S;
    const uint16_t* x;
    int64_t x_sb, x_st, x_sh;
    const int32_t* heads;         /* [nh] device */
    const uint16_t* w;            /* [nh, D, E] bf16 device, or NULL */
    const nkv_rope* rope;         /* host pointer or NULL */
    const int32_t* pairs;         /* [nh, E/2] device or NULL */
    const nkv_camera* camera;     /* host pointer or NULL */
    const int32_t* blocks;        /* [nh, E/8] device or NULL */
    uint16_t* out;
} nkv_reader_rows_args;

int nkv_reader_rows(void* stream, const nkv_reader_rows_args* args);

/*
 * Log-sum-exp merge of two attention partitions (CN/core.py:33-42):
 *   lse = logaddexp(lse_a, lse_b); origin = lse if finite else 0
 *   out = a * exp(lse_a - origin) + b * exp(lse_b - origin)   (fp32, -> bf16)
 * a, b, out: [rows, D] bf16 with row strides (elements); lse_*: [rows] fp32.
 * out may alias a or b.
 */
int nkv_lse_merge(void* stream, int64_t rows, int D,
                  const uint16_t* a, int64_t a_stride, const float* lse_a,
                  const uint16_t* b, int64_t b_stride, const float* lse_b,
                  uint16_t* out, int64_t out_stride, float* lse_out);

/*
 * HY's two history branches merged into the native output with their value
 * lift fused in (HYP:883-1014).  native, low and the LSEs hold 2B batch
 * items: items 0 .. B are the Main branch, items B .. 2B the PRoPE branch.
 *   Main  (b < B):  h_o = sum_k low[b,h,q,k] main_lift[h,k,o]            o < 128
 *   PRoPE (b >= B): h_(4j+c) = sum_k low[b,h,q,4k+c] prope_mix[h,k,j]    j < 32, c < 4
 *   m = max(native_lse, history_lse); wn = exp(native_lse - m), wh = exp(history_lse - m)
 *   out[b,h,q,:] = (native wn + h wh) / (wn + wh)          (fp32, -> bf16 once)
 * low_dim is 32, 64 or 96 (HYP:1834-1835).  All tensors bf16 (uint16_t
 * bits) except the fp32 LSEs; strides in elements; out is contiguous
 * [2B, H, Q, 128] and may not alias an input.
 */
typedef struct nkv_lift_combine_args {
    int B, H, Q, low_dim;
    const uint16_t* native;       /* [2B, H, Q, 128] */
    int64_t n_sb, n_sh, n_sq, n_sd;
    const float* native_lse;      /* [2B, H, Q] */
    int64_t nl_sb, nl_sh, nl_sq;
    const uint16_t* low;          /* [2B, H, Q, low_dim] */
    int64_t l_sb, l_sh, l_sq, l_sd;
    const uint16_t* main_lift;    /* [H, low_dim, 128] */
    int64_t ml_sh, ml_sk, ml_so;
    const uint16_t* prope_mix;    /* [H, low_dim / 4, 32] */
    int64_t pm_sh, pm_sk, pm_so;
    const float* history_lse;     /* [2B, H, Q] */
    int64_t hl_sb, hl_sh, hl_sq;
    uint16_t* out;                /* [2B, H, Q, 128] contiguous */
} nkv_lift_combine_args;

int nkv_lift_lse_combine(void* stream, const nkv_lift_combine_args* args);

/*
 * LingBot's finish of one reader group (LBF:10-46): merge the group's lifted
 * low output into the native output of its heads and scatter the rows to
 * the native head index heads[g].  For group head g, native head hd = heads[g]:
 *   x = native_lse[b,hd,s], z = low_lse[b,g,s]
 *   l = (x == z and |x| = inf) ? x : max(x, z) + log1p(exp(-|x - z|))
 *   origin = l if finite else 0
 *   v = lifted[b,g,s,:]  (+ mean[b,hd,:] - projected[b,g,:] with the value-mean
 *                          correction, LingBot codec_native_attention.py:779-785)
 *   result[b,hd,s,:] = native[b,hd,s,:] exp(x - origin) + v exp(z - origin)
 * in fp32 with one bf16 rounding.  native, lifted, result bf16; the LSEs, mean
 * and projected fp32; mean and projected both set or both NULL.  result may
 * alias native (each element is read before it is written).  A heads entry
 * outside [0, H_native) writes nothing for that group head.
 */
typedef struct nkv_finish_args {
    int B, H_native, H_group, S, D;
    const uint16_t* native;       /* [B, H_native, S, D] */
    int64_t a_sb, a_sh, a_ss, a_sd;
    const float* native_lse;      /* [B, H_native, S] */
    int64_t la_sb, la_sh, la_ss;
    const uint16_t* lifted;       /* [B, H_group, S, D] */
    int64_t b_sb, b_sh, b_ss, b_sd;
    const float* low_lse;         /* [B, H_group, S] */
    int64_t lb_sb, lb_sh, lb_ss;
    const int32_t* heads;         /* [H_group] native head of each group head */
    const float* mean;            /* [B, H_native, D] or NULL */
    int64_t m_sb, m_sh, m_sd;
    const float* projected;       /* [B, H_group, D] or NULL */
    int64_t p_sb, p_sh, p_sd;
    uint16_t* result;             /* [B, H_native, S, D] */
    int64_t y_sb, y_sh, y_ss, y_sd;
} nkv_finish_args;

int nkv_finish(void* stream, const nkv_finish_args* args);

#ifdef __cplusplus
}
#endif

#endif /* NANOKV_H */
