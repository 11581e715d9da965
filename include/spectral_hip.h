/*
 * spectral_hip.h -- C ABI of the MI355X (gfx950) spectral KV-cache library.
 *
 * The library replaces the compute path of unsloth-spectral:
 *   - decode attention over the three-tier cache
 *       unsloth_spectral/kernels/spectral_attention.py:684-857  (absolute RoPE)
 *       unsloth_spectral/spectral_attention.py:117-349          (distance RoPE)
 *   - block compression: randomized SVD + INT8 quantisation
 *       unsloth_spectral/rsvd.py:28-157
 *       unsloth_spectral/spectral_cache.py:321-407, 452-516
 *   - the tier manager (append, compression at the block boundary)
 *       unsloth_spectral/spectral_cache.py:164-319
 *
 * Conventions
 *   - All tensor arguments are raw device pointers (HBM) plus explicit sizes
 *     and element strides.  No entry point allocates memory: callers pass a
 *     workspace where one is needed (size from the matching *_workspace_size).
 *   - Work is enqueued on the caller's stream (a hipStream_t passed as void*;
 *     NULL = the null stream).  No entry point synchronises the host.
 *   - Return value: SC_OK (0) or a negative SC_ERR_* code; sc_last_error()
 *     returns a thread-local message describing the last failure.
 *   - FP16 tensors are IEEE binary16 ("half").
 */
#ifndef UNSLOTH_SPECTRAL_HIP_H
#define UNSLOTH_SPECTRAL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SC_ABI_VERSION 6

#define SC_OK 0
#define SC_ERR_INVALID (-1)      /* bad argument / shape */
#define SC_ERR_UNSUPPORTED (-2)  /* valid but not implemented for this geometry */
#define SC_ERR_WORKSPACE (-3)    /* workspace too small */
#define SC_ERR_HIP (-4)          /* HIP runtime error */
#define SC_ERR_CAPACITY (-5)     /* tier arrays too small for the request */

/* RoPE alignment of cold keys (tail keys are always rotated at their
 * absolute position, as in both reference paths). */
#define SC_ROPE_ABSOLUTE 0 /* kernels/spectral_attention.py:411-446 */
#define SC_ROPE_DISTANCE 1 /* spectral_attention.py:192-219, d = max(q-p,0) */
#define SC_ROPE_NONE 2     /* no rotation (bandwidth reference only)    */

/* INT8 scale granularity. */
#define SC_QUANT_PER_HEAD 0   /* spectral_cache.py:481-516 (reference)     */
#define SC_QUANT_PER_ROW 1    /* one FP32 scale per token row              */
#define SC_QUANT_PER_TENSOR 2 /* spectral_cache.py:452-479 (fallback path) */

/* Per-sequence device counters: int32 counters[batch][SC_NCOUNTERS]. */
#define SC_CNT_NCOLD 0        /* cold blocks in use                      */
#define SC_CNT_TAIL_HEAD 1    /* ring slot of the oldest tail token      */
#define SC_CNT_TAIL_LEN 2     /* tokens in the FP16 tail                 */
#define SC_CNT_NEXT_POS 3     /* reference current_position              */
#define SC_CNT_TOTAL 4        /* reference total_tokens                  */
#define SC_CNT_COMPRESSIONS 5 /* reference compression_count             */
#define SC_CNT_STATUS 6       /* SC_ERR_CAPACITY after an append that did
                                 not fit the ring (nothing was written);
                                 0 otherwise; cleared by a reset          */
#define SC_NCOUNTERS 8

/*
 * One layer's cache for `batch` independent sequences (the reference keeps
 * one SpectralCache per sequence: spectral_cache.py:346).  Layouts
 * (row-major, innermost last):
 *   codes_k     int8  [batch][kv_heads][max_blocks][block_size][kp_keys]
 *   codes_v     int8  [batch][kv_heads][max_blocks][kp_values][block_size]
 *   scales_k/v  fp32  [batch][kv_heads][max_blocks][block_size]  (PER_ROW)
 *                     [batch][kv_heads][max_blocks]              (otherwise)
 *   minmax_k/v  fp32  [batch][kv_heads][max_blocks][2]  reference [min,max]
 *   vnorm       fp32  [batch][kv_heads][max_blocks]     2^-e, e = exponent
 *                     of the block's largest V scale (decode prescale)
 *   basis_k     fp16  [batch][kv_heads][max_blocks][head_dim][kp_keys]
 *   basis_v     fp16  [batch][kv_heads][max_blocks][head_dim][kp_values]
 *   block_start int32 [batch][max_blocks]   absolute position of row 0
 *   tail_k/v    fp16  [batch][kv_heads][tail_capacity][head_dim] (ring,
 *                     pre-RoPE keys as in spectral_cache.py:172)
 *   tail_pos    int32 [batch][tail_capacity]
 *   counters    int32 [batch][SC_NCOUNTERS]
 * kp_* are the ranks padded to 16, 32 or 64; padded code columns and basis
 * rows are zero.
 */
typedef struct ScTierDesc {
  int32_t batch, kv_heads, head_dim, block_size;
  int32_t k_keys, k_values;   /* logical ranks                      */
  int32_t kp_keys, kp_values; /* storage ranks (16, 32 or 64)       */
  int32_t max_blocks, tail_capacity, granularity;
  int8_t* codes_k;
  int8_t* codes_v;
  float* scales_k;
  float* scales_v;
  float* minmax_k;
  float* minmax_v;
  float* vnorm;
  void* basis_k;
  void* basis_v;
  int32_t* block_start;
  void* tail_k;
  void* tail_v;
  int32_t* tail_pos;
  int32_t* counters;
} ScTierDesc;

/*
 * Decode attention for one query token per sequence.
 * Replaces spectral_attention_decode (kernels/spectral_attention.py:684-857,
 * rope_mode = SC_ROPE_ABSOLUTE) and spectral_attention_forward
 * (spectral_attention.py:117-349, rope_mode = SC_ROPE_DISTANCE).
 *   q          fp16 [batch][q_heads][head_dim] (post-RoPE), element strides
 *   cos/sin    fp16 [rope_len][head_dim] RoPE tables (row stride rope_stride)
 *   query_pos  int32 [batch] device array (int64 with query_pos_i64 != 0), or
 *              NULL to use query_pos_scalar
 *   mask       optional uint8 keep-mask (0 = drop, reference
 *              spectral_attention.py:284-285) indexed [b][h][token] in
 *              cache order (cold blocks, then tail); NULL = no mask
 *   out        fp16 [batch][q_heads][head_dim]
 *   logits_out optional fp32 [batch][q_heads][...] = score * scale in cache
 *              order (testing aid); NULL = not written
 *   grid_blocks: cold-block slots scanned per sequence (>= every
 *              counters[b][SC_CNT_NCOLD]); grid_tail: tail tokens scanned
 *              (>= every counters[b][SC_CNT_TAIL_LEN]).
 * halves_equal != 0 asserts cos[:, :D/2] == cos[:, D/2:] (HF tables) and
 * lets the kernel read half rows.
 * split: workgroups per cold block, a power of two dividing block_size/64
 *   (each takes that share of the block's 64-token ranges); 0 = chosen from
 *   the grid size (small batches split their blocks to fill the GPU).  The
 *   split sets the order in which partial results are summed: results with
 *   equal splits are bit-identical for a sequence whatever else is in the
 *   batch; different splits agree to fp32 rounding.  The reference's
 *   TritonSpectralConfig (kernels/spectral_attention.py:50-65) is its
 *   launch-configuration counterpart.
 */
typedef struct ScDecodeArgs {
  const ScTierDesc* tier;
  int32_t q_heads;
  int32_t rope_mode;
  int32_t grid_blocks;
  int32_t grid_tail;
  float scale;
  const void* q;
  int64_t q_stride_b, q_stride_h;
  const void* cos;
  const void* sin;
  int64_t rope_stride;
  int32_t rope_len;
  int32_t halves_equal;
  const int32_t* query_pos;
  int32_t query_pos_scalar;
  const uint8_t* mask;
  int64_t mask_stride_b, mask_stride_h;
  void* out;
  int64_t out_stride_b, out_stride_h;
  float* logits_out;
  int64_t logits_stride_b, logits_stride_h;
  int32_t split;
  int32_t query_pos_i64;  /* nonzero: query_pos points to int64_t[batch] (a model's
                             position ids as they are); 0: int32_t[batch] */
} ScDecodeArgs;

int sc_decode_workspace_size(const ScDecodeArgs* args, size_t* bytes);
int sc_decode_attn(const ScDecodeArgs* args, void* workspace, size_t workspace_bytes,
                   void* stream);
/*
 * sc_decode_attn without a caller workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The partial records live in a
 * library-owned device array of SC_DECODE_SCRATCH_BYTES per GPU (held until
 * the process ends); a call whose records need more (sc_decode_workspace_size)
 * fails with SC_ERR_WORKSPACE.  Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU (different streams or host
 * threads) race and must be serialised by the caller.  Results equal
 * sc_decode_attn's bit for bit.
 */
#define SC_DECODE_SCRATCH_BYTES (32u << 20)
int sc_decode_attn_noalloc(const ScDecodeArgs* args, void* stream);


/*
 * Scores of one block against every query head, absolute RoPE
 * (spectral_score_forward, kernels/spectral_attention.py:375-453):
 *   scores[b][h][t] = fp16( sum_i (R^-1_{start+t} q[b][h]) . basis_k[g][i]
 *                           * coeffs_k[g][t][i] ),  g = h / (q_heads/kv_heads)
 * with the inverse rotation in fp16 elementwise arithmetic as the
 * reference's _apply_inverse_rope (:340-372; halves of cos/sin as given)
 * and the products summed in fp32.
 *   q        fp16 [batch][q_heads][head_dim], element strides (16-byte rows)
 *   coeffs_k fp16 [kv_heads][tokens][rank] (dequantised coefficients)
 *   basis_k  fp16 [kv_heads][rank][head_dim] (16-byte aligned)
 *   cos/sin  fp16 [rope_len][head_dim], row stride rope_stride; key
 *            positions start_position .. start_position + tokens - 1 must
 *            lie inside the tables
 *   scores   fp16 [batch][q_heads][tokens]
 * Supported: head_dim 64 or 128, rank <= 64.
 */
int sc_block_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t q_heads,
                    const void* coeffs_k, const void* basis_k, int32_t kv_heads, int32_t tokens, int32_t rank,
                    int32_t head_dim, const void* cos, const void* sin, int64_t rope_stride, int32_t rope_len,
                    int32_t start_position, void* scores, void* stream);

/*
 * Values of one block (spectral_value_forward,
 * kernels/spectral_attention.py:544-601):
 *   out[b][h] = fp16( (attn[b][h] . coeffs_v[g]) . basis_v[g] ), fp32 sums
 *   attn     fp32 [batch][q_heads][tokens], element strides
 *   coeffs_v fp16 [kv_heads][tokens][rank], basis_v fp16 [kv_heads][rank][head_dim]
 *   out      fp16 [batch][q_heads][head_dim]
 * Supported: head_dim 64 or 128, rank <= 64.
 */
int sc_block_values(const float* attn, int64_t attn_stride_b, int64_t attn_stride_h, int32_t batch,
                    int32_t q_heads, const void* coeffs_v, const void* basis_v, int32_t kv_heads, int32_t tokens,
                    int32_t rank, int32_t head_dim, void* out, void* stream);

/*
 * Query rotation of a decode or prefill step: what the reference's
 * apply_rotary_pos_emb (integration.py:428-465) computes for the queries
 * where its decode caller rotates them (integration.py:610-613), in one
 * launch instead of five elementwise tensor ops:
 *   out = x * cos + rotate_half(x) * sin,  rotate_half(x) = (-x2, x1),
 * each product and the sum rounded to fp16 in that order (bit-identical to
 * the fp16 tensor expression).
 *   x        fp16 [batch][heads][tokens][head_dim], element strides
 *   cos/sin  fp16 [batch][tokens][head_dim], element strides (cs_stride_b = 0
 *            shares one set of rows across the batch)
 *   out      fp16 [batch][heads][tokens][head_dim], contiguous
 * Rows 16-byte aligned (strides multiples of 8).  Supported: head_dim a
 * multiple of 16 in [16, 256].
 */
int sc_rope_rotate(const void* x, int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_t, const void* cos,
                   const void* sin, int64_t cs_stride_b, int64_t cs_stride_t, int32_t batch, int32_t heads,
                   int32_t tokens, int32_t head_dim, void* out, void* stream);

/*
 * Batched block compression: randomized SVD (rsvd.py:74-157, k = rank,
 * oversampling, n_iter) of `count` matrices [rows][cols] (fp16, fp32 or
 * bf16 per m_dtype; computed in fp32 like rsvd.py:79-81), then
 * coeffs = U*S (spectral_cache.py:387) quantised to INT8 and basis = Vh in
 * fp16.  Matrix i = (i / inner, i % inner) is read from
 *   m + (i/inner)*m_stride_outer + (i%inner)*m_stride_inner, rows m_stride_row
 * (element strides; rows 16-byte aligned).
 * omega: fp32 [count][cols][r] Gaussian sketch (r = min(rank+oversample,
 * rows, cols)); NULL = draw it on the device from `seed` (Philox4x32-10 +
 * Box-Muller).  Outputs use the same two-level indexing with their strides:
 *   codes  int8 : coeff_major=0 -> [rows][kp], 1 -> [kp][rows]
 *   scales fp32 : [rows] (PER_ROW) or [1]
 *   minmax fp32 : [2] (may be NULL); vnorm fp32 : [1] (may be NULL)
 *   basis  fp16 : basis_dmajor=1 -> [cols][kp], 0 -> [kp][cols]
 * Optional fp32 testing outputs (NULL = skipped): coeffs [count][rows][rank],
 * svals [count][rank], vh [count][rank][cols], omega_out [count][cols][r].
 * row_weights (NULL = unweighted): fp32 [rows] per matrix, indexed like the
 * outputs (row_weights + (i/inner)*stride_outer + (i%inner)*stride_inner; a
 * stride of 0 shares one vector).  Attention-weighted compression
 * (spectral_cache.py:351-393, `_compress_tensor` with attention_weights):
 * w = sqrt(a / mean(a)), the SVD runs on diag(w) M (products in fp32 on the
 * VALU for every input type), and the coefficients are divided by w before
 * quantisation.  Weights must be positive (a zero weight divides by zero,
 * as in the reference).
 * Supported: rows <= 512 (multiple of 64), cols in {64, 128},
 * rank + oversample <= 40.
 */
#define SC_DTYPE_F16 0
#define SC_DTYPE_F32 1
#define SC_DTYPE_BF16 2

typedef struct ScCompressArgs {
  int32_t count, inner;
  int32_t rows, cols, rank, oversample, n_iter, kp, granularity;
  int32_t coeff_major, basis_dmajor;
  int32_t m_dtype; /* SC_DTYPE_*: element type of m */
  const void* m;
  int64_t m_stride_outer, m_stride_inner, m_stride_row;
  const float* omega;
  uint64_t seed;
  int8_t* codes;
  int64_t codes_stride_outer, codes_stride_inner;
  float* scales;
  int64_t scales_stride_outer, scales_stride_inner;
  float* minmax;
  int64_t minmax_stride_outer, minmax_stride_inner;
  float* vnorm;
  int64_t vnorm_stride_outer, vnorm_stride_inner;
  void* basis;
  int64_t basis_stride_outer, basis_stride_inner;
  float* coeffs_out;
  float* svals_out;
  float* vh_out;
  float* omega_out;
  const float* row_weights;
  int64_t row_weights_stride_outer, row_weights_stride_inner;
} ScCompressArgs;

int sc_rsvd_compress(const ScCompressArgs* args, void* stream);

/*
 * INT8 symmetric quantisation of fp32 x [groups][rows][cols]
 * (spectral_cache.py:452-516): PER_HEAD -> one scale per group,
 * PER_ROW -> one per row, PER_TENSOR -> one in total.
 * scale = max(absmax, 1e-8)/127 (IEEE), code = round_half_even(x/scale).
 * codes int8 like x; scales fp32 [groups] / [groups][rows] / [1];
 * minmax fp32 [groups][2] (may be NULL).
 */
int sc_quantize_int8(const float* x, int64_t groups, int64_t rows, int64_t cols,
                     int32_t granularity, int8_t* codes, float* scales, float* minmax,
                     void* stream);

/*
 * Append t_new tokens to every sequence's FP16 tail (spectral_cache.py:164-232):
 *   k_new, v_new fp16 [batch][kv_heads][t_new][head_dim] with element
 *   strides (stride_b, stride_h, stride_t; innermost contiguous);
 *   positions int32 [batch][t_new] (NULL = continue from NEXT_POS).
 * flags:
 *   SC_APPEND_RESET        every sequence starts a new generation: its
 *                          counters are cleared before the rows are written
 *                          (the caller detected the restart, as the
 *                          reference does on the host, :176-189);
 *   SC_APPEND_DETECT_RESET the device detects it per sequence: a first
 *                          position below NEXT_POS resets that sequence;
 *   SC_APPEND_POS_I64      positions points to int64 [batch][t_new] (a
 *                          model's position ids as they are).
 * Fails with SC_ERR_CAPACITY (before launching) if t_new exceeds the ring.
 * On the device, a sequence whose tail would exceed tail_capacity gets
 * nothing written, keeps its counters and has SC_CNT_STATUS set to
 * SC_ERR_CAPACITY (the reference grows its tail with torch.cat and never
 * overflows; here the caller sizes the ring or compresses first).
 */
#define SC_APPEND_DETECT_RESET 1
#define SC_APPEND_RESET 2
#define SC_APPEND_POS_I64 4
int sc_tier_append(const ScTierDesc* tier, const void* k_new, const void* v_new,
                   int64_t stride_b, int64_t stride_h, int64_t stride_t,
                   const int32_t* positions, int32_t t_new, int32_t flags, void* stream);

/*
 * Compress every full block of every sequence's tail into the next cold
 * slots (spectral_cache.py:243-319), K with rank k_keys and V with k_values,
 * then advance NCOLD / TAIL_HEAD / TAIL_LEN / COMPRESSIONS on the device.
 * max_new_blocks bounds the blocks compressed per sequence in this call
 * (grid size); sequences with fewer full blocks compress what they have.
 * Compression happens only where counters say a block is full, so the
 * call may be enqueued speculatively.  seed drives the Gaussian sketch
 * (block j of sequence b, head h, K/V get distinct Philox streams).
 */
int sc_tier_compress(const ScTierDesc* tier, int32_t max_new_blocks, int32_t n_iter,
                     int32_t oversample, uint64_t seed, void* stream);

/*
 * Dequantise cold blocks [first, first+count) of every sequence into fp16
 * K/V [batch][kv_heads][count*block_size][head_dim] (get_kv,
 * spectral_cache.py:557-612; reference coefficients are fp16(code*scale)).
 */
int sc_tier_dequant(const ScTierDesc* tier, int32_t first, int32_t count, void* k_out,
                    void* v_out, void* stream);

/*
 * Prefill attention: t_q query tokens per sequence attend over every tier
 * of the cache (cold blocks and FP16 tail) with a causal mask (a key is
 * kept iff its position <= the query's position), without materialising
 * keys or values.  Replaces the reference's prefill path
 * (integration.py:292-346: get_kv, apply_rope at the keys' absolute
 * positions with the first half of the cos/sin rows, dense fp16 attention,
 * softmax in fp32).
 *   q          fp16 [batch][q_heads][t_q][128] post-RoPE, element strides
 *              (16-byte aligned rows)
 *   query_pos  int32 [batch][t_q] absolute positions (row stride
 *              query_pos_stride_b)
 *   cos/sin    fp16 [rope_len][128] (row stride rope_stride; only the first
 *              64 columns are read; positions >= rope_len read the last row,
 *              so the tables must cover every cached position)
 *   out        fp16 [batch][q_heads][t_q][128], element strides
 * Supported: head_dim 128, 4 query heads per KV head, padded ranks 16/32/64,
 * block_size a multiple of 16.
 */
typedef struct ScPrefillArgs {
  const ScTierDesc* tier;
  int32_t q_heads;
  int32_t t_q;
  float scale;
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_t;
  const int32_t* query_pos;
  int64_t query_pos_stride_b;
  const void* cos;
  const void* sin;
  int64_t rope_stride;
  int32_t rope_len;
  void* out;
  int64_t out_stride_b, out_stride_h, out_stride_t;
} ScPrefillArgs;

int sc_prefill_attn(const ScPrefillArgs* args, void* stream);

/*
 * Wire format of one cold block of one sequence, for offload and
 * checkpoints.  The reference has no serialised form: its SpectralBlock
 * (spectral_cache.py:20-46) lives only as torch tensors, and
 * get_memory_stats (spectral_cache.py:614-655) only counts their bytes.
 * A record is this 64-byte header followed by eight sections, each at a
 * 16-byte aligned offset from the record start (offsets[] below):
 *   0 codes_k   int8 [kv_heads][block_size][kp_keys]
 *   1 codes_v   int8 [kv_heads][kp_values][block_size]
 *   2 scales_k  fp32 [kv_heads][block_size] (PER_ROW) or [kv_heads]
 *   3 scales_v  fp32 likewise
 *   4 basis_k   fp16 [kv_heads][head_dim][kp_keys]
 *   5 basis_v   fp16 [kv_heads][head_dim][kp_values]
 *   6 minmax    fp32 [2][kv_heads][2] (K, then V; reference [min, max])
 *   7 vnorm     fp32 [kv_heads]
 * All fields little-endian; record_bytes is a multiple of 16, so records
 * follow each other without padding.
 */
#define SC_BLOCK_MAGIC 0x31424353u /* "SCB1" */
#define SC_BLOCK_VERSION 1
#define SC_BLOCK_SECTIONS 8
typedef struct ScBlockHeader {
  uint32_t magic;
  uint16_t version, header_bytes;
  uint32_t record_bytes;
  uint16_t kv_heads, head_dim, block_size;
  uint16_t k_keys, k_values, kp_keys, kp_values;
  uint8_t granularity, reserved;
  int32_t start_position;
  uint32_t offsets[SC_BLOCK_SECTIONS];
} ScBlockHeader;

/* Bytes of one block record for this tier geometry (host only, no GPU). */
size_t sc_block_record_bytes(const ScTierDesc* tier);

/*
 * Pack cold blocks [first_block, first_block + n_blocks) of sequence `seq`
 * into n_blocks consecutive records at dst (device memory, 16-byte
 * aligned, >= n_blocks * sc_block_record_bytes bytes), headers included.
 * The blocks must be in use (checked against nothing on the device: the
 * caller knows its counters).
 */
int sc_tier_pack(const ScTierDesc* tier, int32_t seq, int32_t first_block, int32_t n_blocks, void* dst,
                 size_t dst_bytes, void* stream);

/*
 * Unpack n_blocks records at src (device memory, 16-byte aligned) into cold
 * slots [first_block, first_block + n_blocks) of sequence `seq`: codes,
 * scales, bases, minmax, vnorm and block_start (the record's
 * start_position); NCOLD becomes at least first_block + n_blocks.  Every
 * header is checked on the device against the tier geometry first; if any
 * does not match, nothing is written and *status (device int32, cleared by
 * this call) receives SC_ERR_INVALID.  *status is 0 when the records were
 * taken.
 */
int sc_tier_unpack(const ScTierDesc* tier, int32_t seq, int32_t first_block, int32_t n_blocks,
                   const void* src, size_t src_bytes, int32_t* status, void* stream);

const char* sc_last_error(void);
int sc_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* UNSLOTH_SPECTRAL_HIP_H */
