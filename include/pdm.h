/*
 * pdm.h — C ABI of the MI355X (gfx950) embedding-lookup and OneTrans
 * interaction forward path.
 *
 * Every entry point is extern "C", takes plain pointers and sizes, never
 * throws, and returns a pdm_status (0 = OK, < 0 = error).  The text of the
 * last error on the calling thread is available through pdm_last_error().
 * All device work is enqueued on the caller's HIP stream; no entry point
 * synchronises the host with the device except where stated.
 *
 * Pointers documented as "device" must point at memory of the current HIP
 * device.  Inputs are never written.  Outputs are written completely.
 */
#ifndef PDM_H_
#define PDM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pdm_stream_t; /* == hipStream_t */

typedef enum {
  PDM_OK = 0,
  PDM_ERR_INVALID = -1,     /* bad argument (shape, dtype, null pointer, size) */
  PDM_ERR_UNSUPPORTED = -2, /* valid but not implemented combination */
  PDM_ERR_HIP = -3,         /* a HIP runtime call failed */
  PDM_ERR_WORKSPACE = -4    /* workspace too small */
} pdm_status;

typedef enum {
  PDM_F32 = 0,
  PDM_F16 = 1,
  PDM_BF16 = 2,
  /* int8 rowwise: each row is [fp16 scale][fp16 bias][dim x uint8], the row
   * stride is row_bytes (>= 4 + dim, multiple of 4).  Decode of element d:
   * float(q[d]) * float(scale) rounded to fp32, then + float(bias) rounded
   * to fp32 (two roundings, no fused multiply-add). */
  PDM_I8_SB_F16 = 3
} pdm_dtype;

typedef enum { PDM_POOL_SUM = 0, PDM_POOL_MEAN = 1 } pdm_pooling;

/* Version of this ABI (major * 10000 + minor * 100 + patch). */
int32_t pdm_abi_version(void);

/* Copies the last error message of the calling thread into buf (NUL
 * terminated, truncated to n bytes).  Returns the full message length. */
size_t pdm_last_error(char* buf, size_t n);

/* ------------------------------------------------------------------------
 * Table-batched pooled embedding forward.
 *
 * Replaces the forward of TorchRec EmbeddingBagCollection
 * (primus_dlrm/models/embedding.py:118-120,151; primus_dlrm/models/dlrm.py:147)
 * and of FBGEMM's table-batched embedding op op(indices, offsets) -> [B, sum D]
 * (tests/test_fbgemm_tbe.py:23-35,52-65), including the masked sum/mean
 * pooling written out at primus_dlrm/models/sharded_embedding.py:220-227 and
 * the padding-id filter of _build_pooled_kjt (embedding.py:179-204).
 * ------------------------------------------------------------------------ */

typedef struct {
  int64_t rows;           /* number of rows in the table */
  int64_t weights_offset; /* byte offset of row 0 inside the weights buffer */
  int32_t dim;            /* embedding dim (multiple of 4) */
  int32_t dtype;          /* pdm_dtype of the stored rows */
  int32_t pooling;        /* pdm_pooling */
  int32_t row_bytes;      /* byte stride between rows; 0 = dense default */
  int32_t out_offset;     /* first output column of this table */
  int32_t reserved;
} pdm_table_desc;

typedef struct pdm_tbe_plan_s* pdm_tbe_plan;

/* Validates the table list, uploads its metadata to the current device and
 * groups tables by (dtype, dim) for launch.  Synchronous (one small copy). */
int pdm_tbe_plan_create(const pdm_table_desc* tables, int32_t num_tables,
                        pdm_tbe_plan* plan_out);
int pdm_tbe_plan_destroy(pdm_tbe_plan plan);
/* Sum of dims = number of output columns the plan writes (max out_offset+dim). */
int64_t pdm_tbe_plan_total_dim(pdm_tbe_plan plan);

/* weights:     device, base of all tables (byte addressed by weights_offset)
 * indices:     device, int32 or int64 (index_bits = 32 | 64), num_indices long
 * offsets:     device, int64 [T * B + 1], table-major: bag (t, b) is
 *              indices[offsets[t*B+b] : offsets[t*B+b+1]]
 * padding_idx: an index equal to it is skipped and not counted (negative =
 *              no padding id: every index is pooled or flagged)
 * out:         device, [B, out_row_stride] of out_dtype (F32 | F16 | BF16)
 * err_flag:    optional device int32; set to 1 when an index is outside
 *              [0, rows) (such indices are skipped, never read) or a bag's
 *              offsets are not monotone / exceed num_indices.
 * An empty bag (or one holding only padding) pools to 0 for sum and mean.
 * Mean divides the fp32 sum by the count of pooled indices. */
int pdm_tbe_pooled_fwd(pdm_tbe_plan plan, const void* weights,
                       const void* indices, int32_t index_bits,
                       int64_t num_indices, const int64_t* offsets,
                       int64_t batch_size, int64_t padding_idx, void* out,
                       int32_t out_dtype, int64_t out_row_stride,
                       int32_t* err_flag, pdm_stream_t stream);

/* Quantizes fp32 rows [rows, dim] (device) into int8 rowwise rows
 * (PDM_I8_SB_F16 layout, row stride row_bytes) on the device:
 * bias = fp16(min row), scale = fp16((max - bias) / 255) (1 when the range is
 * 0), q = clamp(rint((x - bias) * (1 / scale)), 0, 255). */
int pdm_int8_rowwise_quantize(const float* src, int64_t rows, int32_t dim,
                              void* dst, int32_t row_bytes,
                              pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * Pooled TBE backward with the embedding optimizer fused in.
 *
 * Replaces the backward of the fused-optimizer table-batched embedding that
 * TorchRec builds for an EmbeddingBagCollection whose weights were tagged by
 * _apply_optimizer_in_backward (primus_dlrm/distributed/wrapper.py:151-174):
 * FBGEMM's EmbOptimType.ADAM for torch.optim.Adam (the default,
 * primus_dlrm/config.py:411-418) and EXACT_ROWWISE_ADAGRAD for
 * torchrec.optim.RowWiseAdagrad with WeightDecayMode.L2
 * (fbgemm_gpu 2026.4.29, scripts/launch_slurm_docker.sh:402, not vendored).
 *
 * The gradient of a table row is the sum, over every lookup of that row in
 * the batch, of grad_out[b, out_offset : out_offset + dim] of the lookup's bag
 * (times 1 / count for mean pooling, count = pooled indices of the bag);
 * padding ids and out-of-range ids contribute nothing.  Only rows looked up
 * in the batch are updated (sparse update), each exactly once.
 *
 * Row space: the plan's distinct tables (slots with equal weights_offset,
 * rows, dim, dtype and row_bytes are one table) are numbered group by group
 * ((dtype, dim) groups in first-appearance order) and in table order inside a
 * group; row r of a table has row id pdm_tbe_plan_row_offset(slot) + r.
 * Row-wise optimizer state is one fp32 per row id.
 * ------------------------------------------------------------------------ */

typedef enum {
  PDM_OPT_ADAM = 0,            /* FBGEMM ADAM: per-element m, v */
  PDM_OPT_ROWWISE_ADAGRAD = 1, /* FBGEMM EXACT_ROWWISE_ADAGRAD: one sum per row */
  PDM_OPT_NONE = 2             /* gradient only (pdm_tbe_backward_sparse_grad) */
} pdm_optimizer;

typedef enum { PDM_WD_NONE = 0, PDM_WD_L2 = 1 } pdm_weight_decay_mode;

typedef struct {
  int32_t optimizer;         /* pdm_optimizer */
  int32_t weight_decay_mode; /* row-wise Adagrad: PDM_WD_NONE | PDM_WD_L2 */
  float learning_rate;
  float eps;
  float beta1;               /* Adam */
  float beta2;               /* Adam */
  float weight_decay;        /* Adam: decoupled term lr * wd * w */
  int32_t reserved;
  int64_t step;              /* Adam: 1-based count of this update */
} pdm_optim_params;

/* Rows of the plan's row space, and the row id of row 0 of a slot's table
 * (-1 on a bad argument). */
int64_t pdm_tbe_plan_total_rows(pdm_tbe_plan plan);
int64_t pdm_tbe_plan_row_offset(pdm_tbe_plan plan, int32_t slot);

/* Where each slot's table keeps its row-wise optimizer state: row r of slot
 * t's table uses entry state_row_offsets[t] + r (host array, one per slot;
 * -1 keeps the default, the row id).  Lets several plans over one set of
 * tables (e.g. a collection's pooled features and its S-token gather) share
 * one state buffer.  Slots of one table need equal offsets.  Synchronous. */
int pdm_tbe_plan_set_state_offsets(pdm_tbe_plan plan,
                                   const int64_t* state_row_offsets);

/* Device workspace bytes the backward needs for num_indices lookups over
 * batch_size bags per slot. */
int64_t pdm_tbe_backward_workspace_size(pdm_tbe_plan plan, int64_t num_indices,
                                        int64_t batch_size);

/* Fused backward + optimizer update, in place.
 * weights:   device fp32 base (every slot PDM_F32, row_bytes == 4 * dim,
 *            weights_offset a multiple of 16)
 * momentum1: Adam: fp32 buffer laid out like weights (same byte offsets);
 *            row-wise Adagrad: fp32 [pdm_tbe_plan_total_rows]
 * momentum2: Adam: like momentum1; row-wise Adagrad: unused (may be NULL)
 * indices, index_bits, num_indices, offsets, batch_size, padding_idx: as in
 *            pdm_tbe_pooled_fwd for the same batch
 * grad_out:  device fp32 [B, grad_row_stride], d(loss)/d(pooled output)
 *            (grad_row_stride and every out_offset multiples of 4,
 *            16-byte aligned base)
 * workspace: device, >= pdm_tbe_backward_workspace_size bytes
 * err_flag:  optional device int32, set to 1 on an out-of-range index or
 *            malformed offsets (those entries and bags are skipped; where
 *            non-monotone offsets make two bags share a lookup, that lookup
 *            counts for one of them).
 * The update is deterministic: the same inputs give the same bits. */
int pdm_tbe_backward_fused(pdm_tbe_plan plan, float* weights, float* momentum1,
                           float* momentum2, const void* indices,
                           int32_t index_bits, int64_t num_indices,
                           const int64_t* offsets, int64_t batch_size,
                           int64_t padding_idx, const float* grad_out,
                           int64_t grad_row_stride,
                           const pdm_optim_params* opt, void* workspace,
                           int64_t workspace_bytes, int32_t* err_flag,
                           pdm_stream_t stream);

/* The deduplicated row gradients the fused update consumes (all slots of
 * the plan must share one dim D):
 * row_ids:   device int64 [num_indices]; first *num_unique entries = the
 *            distinct row ids looked up, ascending
 * grad_rows: device fp32 [num_indices, D]; row u = gradient of row_ids[u]
 * num_unique: device int64 scalar. */
int pdm_tbe_backward_sparse_grad(pdm_tbe_plan plan, const void* indices,
                                 int32_t index_bits, int64_t num_indices,
                                 const int64_t* offsets, int64_t batch_size,
                                 int64_t padding_idx, const float* grad_out,
                                 int64_t grad_row_stride, int64_t* row_ids,
                                 float* grad_rows, int64_t* num_unique,
                                 void* workspace, int64_t workspace_bytes,
                                 int32_t* err_flag, pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * Jagged -> padded S-token sequence gather.
 *
 * Replaces the unpooled lookup TorchRec EmbeddingCollection.forward
 * (embedding.py:156-172, onetrans.py:480-509), the per-pool concat of
 * item|artist|album embeddings (onetrans.py:515-520) and the pool concat
 * along the sequence (onetrans.py:553-558), with the host-side jagged->padded
 * step of the data loader (primus_dlrm/data/dataset.py:604-636) moved onto
 * the device.  A pool keeps its last min(len, max_len) events.
 * ------------------------------------------------------------------------ */

#define PDM_SEQ_MAX_POOLS 8
#define PDM_SEQ_MAX_FEATURES 8

typedef enum { PDM_PAD_ROW0 = 0, PDM_PAD_ZERO = 1 } pdm_pad_mode;
typedef enum { PDM_ALIGN_RIGHT = 0, PDM_ALIGN_LEFT = 1 } pdm_align;

typedef struct {
  int32_t num_pools;    /* P <= PDM_SEQ_MAX_POOLS */
  int32_t num_features; /* F <= PDM_SEQ_MAX_FEATURES (tables per event) */
  int32_t dtype;        /* PDM_F32 | PDM_F16 | PDM_BF16, tables and output */
  int32_t pad_mode;     /* pdm_pad_mode; ROW0 = reference (id 0 lookup) */
  int32_t align;        /* pdm_align; RIGHT = reference (left padded) */
  int32_t reserved;
  int64_t batch_size;                         /* B */
  int32_t max_len[PDM_SEQ_MAX_POOLS];         /* padded length per pool */
  int32_t dim[PDM_SEQ_MAX_FEATURES];          /* dim per feature table */
  int64_t rows[PDM_SEQ_MAX_FEATURES];         /* rows per feature table */
  int64_t num_ids[PDM_SEQ_MAX_POOLS];         /* entries in each id array of
                                                 pool p (offsets[p][B] <= it) */
} pdm_seq_desc;

/* tables:  [F] device pointers, dense row-major [rows, dim] of dtype
 * ids:     [P * F] device pointers, int64, pool-major; ids[p*F+f] has
 *          offsets[p][B] entries
 * offsets: [P] device pointers, int64 [B + 1] per pool
 * out:     device, [B, sum_p max_len[p], sum_f dim[f]] of dtype
 * mask:    device, uint8 [B, sum_p max_len[p]] (1 = event, 0 = padding); may
 *          be NULL
 * err_flag: optional device int32, set to 1 on an id outside [0, rows)
 *          (that slot is written as zeros) or bad offsets. */
int pdm_seq_gather_fwd(const pdm_seq_desc* desc, const void* const* tables,
                       const int64_t* const* ids,
                       const int64_t* const* offsets, void* out,
                       uint8_t* mask, int32_t* err_flag, pdm_stream_t stream);

/* Backward of pdm_seq_gather_fwd with the embedding optimizer fused in: the
 * S-token slot (b, s) of feature f is a one-id bag whose gradient is
 * grad_out[b, s, col_f : col_f + dim_f], so every looked-up row (row 0 for a
 * ROW0 padding slot, as the forward reads it) gets the sum of its slots'
 * gradients and one update (replaces the EmbeddingCollection backward of the
 * reference's sequence lookups, onetrans.py:480-520,553-558, under the fused
 * optimizer of distributed/wrapper.py:151-174).
 * plan:      one slot per feature, fp32 tables, sum pooling, slot f's
 *            out_offset = col_f (sum of the earlier dims), rows/dim as desc
 * desc, ids, offsets: as given to the forward (desc->dtype = PDM_F32)
 * grad_out:  device fp32 [B, S, sum dim] (S = sum max_len)
 * weights, momentum1, momentum2, opt, err_flag: as pdm_tbe_backward_fused
 * workspace: >= pdm_tbe_backward_workspace_size(plan, F * B * S, B * S). */
int pdm_seq_gather_backward_fused(pdm_tbe_plan plan, const pdm_seq_desc* desc,
                                  float* weights, float* momentum1,
                                  float* momentum2, const int64_t* const* ids,
                                  const int64_t* const* offsets,
                                  const float* grad_out,
                                  const pdm_optim_params* opt, void* workspace,
                                  int64_t workspace_bytes, int32_t* err_flag,
                                  pdm_stream_t stream);

/* S-token gather fused with the per-pool SequentialTokenizer
 * (primus_dlrm/models/onetrans.py:238-257, one per sequence group at
 * :326-332,553-558) under autocast(bf16): for slot l of pool p of sample b,
 *   raw = concat_f table_f[id_f]         (the gather's placement and padding,
 *                                         as pdm_seq_gather_fwd; bf16, fp32
 *                                         tables rounded to bf16 on load)
 *   h   = bf16(gelu(bf16(raw . W1_p^T + b1_p)))          (exact-erf GELU)
 *   out[b, s0_p + l, :] = float(bf16(h . W2_p^T + b2_p)) + pos_p[l]   (fp32)
 * so the [B, S, sum dim] raw rows never reach memory.  The padding slots of a
 * pool share one raw row, whose MLP runs once.
 * desc:    the gather (dtype PDM_BF16 or PDM_F32; every dim a multiple of 8,
 *          sum of dims = raw_dim in {128, 192, 256, 384}; ROW0 padding needs
 *          rows >= 1)
 * weights: [P]; w1 [d_model, raw_dim], w2 [d_model, d_model], b1, b2
 *          [d_model] bf16 (autocast's casts of the fp32 parameters); pos fp32
 *          [pos_rows >= max_len[p], d_model] or NULL (use_pos_embed = False);
 *          16-byte aligned.  Unused (may be NULL) for pools with max_len 0.
 * out:     fp32, 16-byte aligned; token (b, s) at
 *          out + b * out_sample_stride + s * d_model (e.g. the first S rows of
 *          the block's [B, S + n_ns, d_model] input)
 * d_model: 128, 256 or 384.  mask / err_flag as pdm_seq_gather_fwd (mask
 *          optional).  B * S < 2^31.
 * workspace: 256-byte aligned, >= pdm_seq_tokenize_workspace_size(desc,
 *          d_model) bytes; no initialisation needed; calls sharing one
 *          workspace must not overlap.
 * Streams: the padding rows and the mask are written on the library's own
 * second stream of the device (default priority), forked from `stream` after
 * the first kernel and joined back into it before the call returns, so work
 * queued on `stream` afterwards sees the whole output.  The library makes that
 * stream on a device's first call outside a stream capture; a first call
 * inside a capture runs everything on `stream`.  Under HIP graph capture the
 * fork and join become graph edges. */
typedef struct {
  const uint16_t* w1;
  const uint16_t* b1;
  const uint16_t* w2;
  const uint16_t* b2;
  const float* pos;
  int64_t pos_rows;
} pdm_tokenizer_weights;

int64_t pdm_seq_tokenize_workspace_size(const pdm_seq_desc* desc,
                                        int32_t d_model);

int pdm_seq_tokenize_fwd(const pdm_seq_desc* desc, const void* const* tables,
                         const int64_t* const* ids,
                         const int64_t* const* offsets,
                         const pdm_tokenizer_weights* weights,
                         int32_t d_model, float* out,
                         int64_t out_sample_stride, uint8_t* mask,
                         void* workspace, int64_t workspace_bytes,
                         int32_t* err_flag, pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * OneTrans mixed-parameter interaction block forward (bf16 MFMA).
 *
 * Replaces OneTransBlock.forward(x, mask, q_len, n_s_tokens)
 * (primus_dlrm/models/onetrans.py:207-231) run under autocast(bf16), with
 * RMSNorm (:74-82), MixedAttention (:85-169) and MixedFFN (:172-204).  The
 * mask must be the bottom-right causal pyramid mask of build_pyramid_mask
 * (:62-67), which is the only mask the reference passes (:581-582).
 * ------------------------------------------------------------------------ */

typedef struct {
  int32_t batch;    /* B */
  int32_t d_model;  /* D: 128 or 256 (fused kernels), 384 or 512 (tiled kernels) */
  int32_t n_heads;  /* H (D / H = 64 supported) */
  int32_t n_ns;     /* NS tokens at the end of the sequence */
  int32_t ffn_dim;  /* FFN hidden (multiple of 128) */
  int32_t kv_len;   /* tokens in x */
  int32_t q_len;    /* tokens kept (tail of x), n_ns <= q_len <= kv_len */
  int32_t reserved;
} pdm_block_desc;

typedef struct {
  const float* norm1_w;   /* fp32 [D] */
  const void* s_qkv_w;    /* bf16 [3D, D]  (nn.Linear weight) */
  const void* ns_qkv_w;   /* bf16 [NS, 3D, D] */
  const void* out_w;      /* bf16 [D, D] */
  const float* norm2_w;   /* fp32 [D] */
  const void* s_w1;       /* bf16 [F, D] */
  const void* s_w2;       /* bf16 [D, F] */
  const void* ns_w1;      /* bf16 [NS, F, D] */
  const void* ns_w2;      /* bf16 [NS, D, F] */
} pdm_block_weights;

/* Bytes of device workspace pdm_onetrans_block_fwd needs for desc. */
int64_t pdm_onetrans_block_workspace_size(const pdm_block_desc* desc);

/* x: device fp32 [B, kv_len, D] (the residual stream); y: device fp32
 * [B, q_len, D]; workspace: device, >= pdm_onetrans_block_workspace_size. */
int pdm_onetrans_block_fwd(const pdm_block_desc* desc, const float* x,
                           const pdm_block_weights* w, float* y,
                           void* workspace, int64_t workspace_bytes,
                           pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * OneTrans block stack: the layer loop of OneTransModel._backbone
 * (primus_dlrm/models/onetrans.py:568-582).  Layer l runs OneTransBlock l on
 * the previous layer's output (layer 0 on x, kv_len = desc->kv_len; layer l
 * > 0 with kv_len = the previous layer's q_len) with the pyramid mask and
 * q_len = q_s[l] + n_ns, n_s_tokens = kv_len - n_ns (:574-582); q_s is the
 * schedule of pyramid_schedule (:50-59) or [L_S] * n_layers.  desc gives B,
 * D, H, n_ns, ffn_dim and layer 0's kv_len (its q_len is not read).
 * weights: n_layers layers.  x: device fp32 [B, kv_len, D]; y: device fp32
 * [B, q_s[n_layers-1] + n_ns, D].  One workspace serves every layer (the
 * inner layers' outputs live in it); the intermediate tensors never reach
 * the caller and no per-layer call crosses the ABI.
 * ------------------------------------------------------------------------ */
#define PDM_STACK_MAX_LAYERS 64

/* Bytes of device workspace pdm_onetrans_stack_fwd needs. */
int64_t pdm_onetrans_stack_workspace_size(const pdm_block_desc* desc,
                                          const int32_t* q_s, int32_t n_layers);

int pdm_onetrans_stack_fwd(const pdm_block_desc* desc, const int32_t* q_s,
                           int32_t n_layers, const float* x,
                           const pdm_block_weights* weights, float* y,
                           void* workspace, int64_t workspace_bytes,
                           pdm_stream_t stream);

/* NS-token construction: OneTransModel._build_ns_raw
 * (primus_dlrm/models/onetrans.py:522-532) + AutoSplitTokenizer
 * (onetrans.py:260-276), used at onetrans.py:561-563, under autocast(bf16):
 *   raw[b] = concat(table_f[ids_f[b]] for the scalar features,
 *                   dense_j[b] for the dense parts)            (bf16)
 *   h[b]   = bf16(gelu(bf16(raw[b] . W1^T + b1)))             (N = d * n_ns)
 *   out[b] = float(bf16(h[b] . W2^T + b2)), viewed as [n_ns, d] rows
 * The dense parts are given as computed (the reference's projections
 * dense_projs[name](batch[name]) run before, or the raw feature).
 * ------------------------------------------------------------------------ */

#define PDM_NS_MAX_PARTS 8

typedef struct {
  int32_t num_scalar;   /* scalar feature tables (0..8) */
  int32_t num_dense;    /* dense parts (0..8) */
  int32_t table_dtype;  /* PDM_F32 | PDM_BF16 (all scalar tables) */
  int32_t n_out;        /* N = d_model * n_ns, a multiple of 64 */
  int64_t batch_size;
  int32_t scalar_dim[PDM_NS_MAX_PARTS]; /* >= 1 */
  int64_t scalar_rows[PDM_NS_MAX_PARTS];
  int32_t dense_dim[PDM_NS_MAX_PARTS];  /* any >= 1 */
} pdm_ns_desc;

/* Bytes of device workspace pdm_ns_tokenize_fwd needs. */
int64_t pdm_ns_tokenize_workspace_size(const pdm_ns_desc* desc);

/* tables / ids: [num_scalar] device pointers, ids int64 [B] each (one id per
 * sample; an id outside the table reads zeros and sets err_flag);
 * dense: [num_dense] device pointers to fp32 [B, dense_dim] rows (row stride
 * dense_stride[j] floats); w1 bf16 [N, K] (K = sum of the dims, in the order
 * above), b1 bf16 [N], w2 bf16 [N, N], b2 bf16 [N]; out fp32, sample b's N
 * values at out + b * out_sample_stride (e.g. the n_ns NS rows of the block
 * input).  workspace: 256-byte aligned, pdm_ns_tokenize_workspace_size bytes,
 * no initialisation needed. */
int pdm_ns_tokenize_fwd(const pdm_ns_desc* desc, const void* const* tables,
                        const int64_t* const* ids, const float* const* dense,
                        const int64_t* dense_stride, const uint16_t* w1,
                        const uint16_t* b1, const uint16_t* w2,
                        const uint16_t* b2, float* out,
                        int64_t out_sample_stride, void* workspace,
                        int64_t workspace_bytes, int32_t* err_flag,
                        pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * KeyedJaggedTensor construction on the device (no host synchronisation).
 *
 * Replaces _build_pooled_kjt (primus_dlrm/models/embedding.py:177-204): per
 * feature, mask = ids != padding_idx over a dense [B, L] id matrix, lengths =
 * mask.sum(1), values = ids[mask] (row-major), features concatenated in
 * order; and the key permutation of build_kjt / KJT.permute
 * (primus_dlrm/data/pipeline_batch.py:70-100).  The reference sizes `values`
 * with a host sync; here values are written into a buffer of the known
 * capacity and the exact count is offsets[rows] on the device.
 * ------------------------------------------------------------------------ */

#define PDM_KJT_MAX_FEATURES 64

/* Workspace bytes for num_rows (= keys * batch) lengths. */
int64_t pdm_kjt_workspace_size(int64_t num_rows);

/* ids[f]:    device [B, row_len[f]] int32 / int64 (index_bits), row-major
 * row_len:   host [num_features]
 * values:    device, capacity sum_f B * row_len[f] ids of the same type;
 *            the first offsets[F*B] hold the kept ids, feature-major
 * lengths:   device int32 [F * B]; offsets: device int64 [F * B + 1]
 * padding_idx < 0 keeps every id. */
int pdm_kjt_from_dense(const void* const* ids, const int32_t* row_len,
                       int32_t num_features, int64_t batch_size,
                       int32_t index_bits, int64_t padding_idx, void* values,
                       int32_t* lengths, int64_t* offsets, void* workspace,
                       int64_t workspace_bytes, pdm_stream_t stream);

/* pdm_kjt_from_dense without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The scan's block sums live in a
 * library-owned static device array (512 KiB per device, held until the
 * process ends), so F * B must not exceed PDM_KJT_NOALLOC_MAX_ROWS (larger
 * inputs return PDM_ERR_INVALID), and calls that overlap on one GPU (on
 * different streams) race on that array.  The first call on a device looks
 * up the array's address (hipGetSymbolAddress): under graph capture, make one
 * call on the device before capturing.  Arguments and results are those of
 * pdm_kjt_from_dense. */
#define PDM_KJT_NOALLOC_MAX_ROWS 67108864
int pdm_kjt_from_dense_noalloc(const void* const* ids, const int32_t* row_len,
                               int32_t num_features, int64_t batch_size,
                               int32_t index_bits, int64_t padding_idx,
                               void* values, int32_t* lengths,
                               int64_t* offsets, pdm_stream_t stream);

/* Reorders the keys of a KJT (values, offsets [num_keys * B + 1]): output key
 * k is input key perm[k] (host array, num_out <= PDM_KJT_MAX_FEATURES; keys
 * may repeat or be dropped).  out_values: capacity of the input's values;
 * out_lengths int32 [num_out * B]; out_offsets int64 [num_out * B + 1]. */
int pdm_kjt_permute(const void* values, int32_t index_bits,
                    const int64_t* offsets, int32_t num_keys,
                    int64_t batch_size, const int32_t* perm, int32_t num_out,
                    void* out_values, int32_t* out_lengths,
                    int64_t* out_offsets, void* workspace,
                    int64_t workspace_bytes, pdm_stream_t stream);

/* ------------------------------------------------------------------------
 * Cross-feature ids: xxHash64 of the little-endian concatenation of n int64
 * keys, seeded with salt, modulo table_size (an unsigned 64-bit remainder).
 *
 * Replaces cross_hash_nway / cross_hash_int64 / cross_hash_batch
 * (primus_dlrm/data/hashing.py:23-52,55-69,72-112), which the dataset calls
 * once per event and cross spec (primus_dlrm/data/dataset.py:586-602); the
 * result is the row id of the spec's EmbeddingCollection table
 * (primus_dlrm/config.py:124-160).
 * ------------------------------------------------------------------------ */

#define PDM_CROSS_MAX_KEYS 8

/* keys: host array of num_keys device pointers (2 <= num_keys <= 8), key k of
 * row i at keys[k][i * key_strides[k]]; a stride of 0 broadcasts one value
 * to every row.  out: device int64 [n], every value in [0, table_size).
 * table_size >= 1. */
int pdm_cross_hash_fwd(const int64_t* const* keys, const int64_t* key_strides,
                       int32_t num_keys, int64_t n, uint64_t table_size,
                       uint64_t salt, int64_t* out, pdm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PDM_H_ */
