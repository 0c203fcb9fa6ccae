/*
 * shrimp_hip.h — C ABI of the MI355X (gfx950) Shrimp forward kernels.
 *
 * Every entry point:
 *   - takes plain device pointers (non-owning), sizes and a hipStream_t passed
 *     as `void* stream` (NULL = the null stream);
 *   - allocates nothing, never synchronises the host, and only enqueues work
 *     on `stream`, so it can be captured into a HIP graph;
 *   - returns 0 on success or a negative status; the message of the last
 *     failure on the calling thread is available from shrimp_last_error().
 *
 * Shapes: B positions, N padded cells per position (Npad), S = n_tokens + N
 * sequence rows, C channels, H heads, d = C / H head dim.
 * Activations are bf16 with fp32 accumulation; element strides are given in
 * elements (not bytes).
 */
#ifndef SHRIMP_HIP_H
#define SHRIMP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SHRIMP_ABI_VERSION 1

/* Status codes. */
#define SHRIMP_OK 0
#define SHRIMP_EINVAL (-1)   /* bad argument / unsupported shape */
#define SHRIMP_ELAUNCH (-2)  /* HIP launch error */
/* Checked builds only (libshrimp_hip_check.so, built with SHRIMP_DEBUG=1): a
 * kernel found an input outside its contract (an index past the rows, a length
 * past the sequence). Every launch of such a build is followed by a device
 * synchronisation and a read of the kernels' fault word, so it cannot be
 * captured into a graph; shrimp_last_error names the failed checks. */
#define SHRIMP_ECHECK (-3)

/* Element types for the few entry points that accept several. */
#define SHRIMP_DT_BF16 0
#define SHRIMP_DT_F32 1
#define SHRIMP_DT_F16 2
#define SHRIMP_DT_I64 3
#define SHRIMP_DT_I32 4
#define SHRIMP_DT_U16 5
#define SHRIMP_DT_U8 6

const char* shrimp_last_error(void);
int shrimp_abi_version(void);

/* Tuning / test switches (no counterpart in the reference).
 * shrimp_conv_variant: 0 = automatic conv kernel choice (a position's rows
 * staged in LDS when they fit, 128x128 tiles per wave for the 128-channel
 * 7-tap conv, and for batches of at most half the compute-unit count one
 * 64-row tile per workgroup so a position's rows spread over several; that
 * split repeats the big-tile kernel's arithmetic where the big-tile kernel
 * would serve a large batch, so results do not depend on the batch), 1 = always
 * gather rows from global memory, 2 = LDS-staged rows with small tiles,
 * 3 = as 0 without the small-batch row split; other values only query.
 * Returns the previous setting. Process-wide.
 * shrimp_attn_variant: 0 = automatic (two heads per attention workgroup when
 * their K/V fit the 64 KiB budget, on eight waves at padded head dim 16, else
 * four; one head per workgroup with up to the device's per-workgroup LDS for
 * longer sequences; beyond that the chunked kernel of shrimp_attn_f32 on bf16
 * operands), 1 = one head per workgroup, 2 = two heads on four waves, 3 = the
 * chunked kernel; other values only query. Returns the previous setting.
 * Process-wide.
 * shrimp_max_lds_per_block: LDS bytes one workgroup may allocate on the
 * current device (the staged conv needs (N + 1) * cin_pad * 2). */
int shrimp_conv_variant(int variant);
int shrimp_attn_variant(int variant);
int shrimp_max_lds_per_block(void);

/* Phase stamps (measurement builds only; no counterpart in the reference).
 * In libshrimp_hip_phase.so (built with SHRIMP_PHASE_CLOCK=1) every later
 * launch of the unit's instrumented kernels (unit 0: the big-tile conv and the
 * ConvBlock pair; unit 1: the staged attention) stores the 100 MHz constant
 * clock at its phase boundaries into `stamps` (device memory, 32 uint64 per
 * workgroup, workgroup blockIdx.x + gridDim.x * blockIdx.y, blockIdx.z not
 * told apart; slots 0-7 from the workgroup after a barrier, 16 + 8 k + wave
 * from each wave); unit + 4 also stores the core clock counter of each
 * workgroup stamp at slot + 8 (a second counter read per stamp: take timings
 * from runs without it); NULL stops.
 * Other builds return SHRIMP_EINVAL. Process-wide. */
int shrimp_phase_clock(void* stamps, int unit);

/* ------------------------------------------------------------------------
 * Weight packing (device -> device). MFMA operands are read in fragment
 * order: for K-step ks (32 rows of K) and output block nb (16 outputs), 64
 * lanes x 8 bf16, lane l holding W[k = 32*ks + 8*(l/16) + e][n = 16*nb + l%16].
 *
 * Conv weights (HexNodeConv.weight, (T, cin, cout) fp32, model.py:338) are
 * packed with K = T * cin_pad (tap-major, zero rows for cin <= c < cin_pad).
 * Linear weights (nn.Linear.weight, (out, in) fp32) use K = in, n = out.
 * ---------------------------------------------------------------------- */
size_t shrimp_conv_wpack_bytes(int taps, int cin_pad, int cout);
int shrimp_pack_conv_weight(const float* w, void* packed, int taps, int cin, int cin_pad,
                            int cout, void* stream);
size_t shrimp_linear_wpack_bytes(int in_features, int out_features);
int shrimp_pack_linear_weight(const float* w, void* packed, int in_features, int out_features,
                              void* stream);

/* ------------------------------------------------------------------------
 * Gather-GEMM hex / ray-tap convolution with fused epilogue.
 *
 * Replaces shrimp::hex_conv (packages/shrimp/python/shrimp/_triton_conv.py:93-122),
 * shrimp::hex_conv_ln (_triton_conv.py:198-231), the materialized
 * HexNodeConv.forward (model.py:346-370), ConvBlock.forward (model.py:395-422)
 * and the policy head ShrimpNet._policy_logits (model.py:1011-1020).
 *
 *   acc[r, n] = bias[n] + sum_t sum_c x[b, idx[r, t], c] * W[t, c, n]
 *   y = acc; if ln_w: y = LayerNorm(y) * ln_w + ln_b (fp32 stats, eps)
 *   if relu: y = max(y, 0); y = mask[r] ? y : 0
 *   residual (resid != NULL): out = max(resid[r, n] + gamma[n] * y, 0)
 *   head (head_w != NULL): head_out[r] = mask[r] ? sum_n max(acc,0)*head_w[n] + head_b[0] : 0
 *                          (no activation store)
 *   else out = y.
 * idx values outside [0, N) read as zero rows (the Npad sentinel of the
 * reference). x, resid and out are bf16 with strides (per position, per row);
 * out may alias resid (each row reads only its own residual row); out must not
 * alias x.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* x;
  int64_t x_sb, x_sn;
  const int32_t* idx; /* (B, N, idx_stride) */
  int32_t taps, idx_stride;
  const uint8_t* mask; /* (B, N) */
  const void* w;       /* packed, taps * cin_pad x cout */
  const float* bias;   /* (cout) */
  const float* ln_w;   /* (cout) or NULL */
  const float* ln_b;
  float eps;
  int32_t relu;
  const void* resid;
  int64_t r_sb, r_sn;
  const float* gamma;  /* LayerScale (cout), required with resid */
  const float* head_w; /* (cout) or NULL */
  const float* head_b; /* (1) */
  float* head_out;     /* (B, N) fp32 */
  void* out;
  int64_t o_sb, o_sn;
  int32_t B, N, cin_pad, cout;
} shrimp_conv_args;

int shrimp_hex_conv(const shrimp_conv_args* a, void* stream);

/* ------------------------------------------------------------------------
 * ConvBlock.forward (model.py:395-422) in one launch:
 *   y1  = relu(LN1(conv1(x))) * m ;   out = relu(x + gamma * LN2(conv2(y1)) * m)
 * the same result as shrimp_hex_conv(c1) followed by shrimp_hex_conv(c2) with
 * c2.x = c1's output, but y1 never leaves the workgroup's LDS.
 * c1: x, idx, taps, idx_stride, mask, w, bias, ln_w, ln_b, eps, relu = 1,
 *     B, N, cin_pad, cout (out / resid / head unused);
 * c2: w, bias, ln_w, ln_b, eps, relu = 0, resid = c1.x (same strides),
 *     gamma, out, o_sb, o_sn (x, idx, mask, B, N are taken from c1).
 * out may alias x; out must be 16-byte aligned with o_sb, o_sn multiples of 8
 * (rows leave as 16-byte stores). shrimp_conv_block_supported reports whether a fused
 * kernel exists for the shape (taps 7, 128 -> 128 channels, N <= 512, and
 * the automatic conv variant selected); otherwise shrimp_conv_block returns
 * SHRIMP_EINVAL and the caller runs the two convolutions.
 * ---------------------------------------------------------------------- */
int shrimp_conv_block_supported(int taps, int N, int cin_pad, int cout);
int shrimp_conv_block(const shrimp_conv_args* c1, const shrimp_conv_args* c2, void* stream);

/* Two consecutive ConvBlocks in one launch (no counterpart in the reference,
 * which runs ConvBlock.forward per block, model.py:395-422; the trunk layouts
 * repeat "CC"): shrimp_conv_block(c1, c2) then shrimp_conv_block(c3, c4), with
 * the same result, the first block's output rows handed to the second inside
 * the workgroup instead of read back from HBM. (c1, c2) and (c3, c4) each meet
 * shrimp_conv_block's contract; c3.x must be c2.out (same strides), and c3
 * shares c1's idx, idx_stride, mask, B and N. shrimp_conv_block_pair_supported
 * reports whether the pair fits one workgroup's LDS (else SHRIMP_EINVAL). */
int shrimp_conv_block_pair_supported(int taps, int N, int cin_pad, int cout);
int shrimp_conv_block_pair(const shrimp_conv_args* c1, const shrimp_conv_args* c2,
                           const shrimp_conv_args* c3, const shrimp_conv_args* c4, void* stream);

/* ------------------------------------------------------------------------
 * Dense row GEMM with fused prologue / epilogue (the nn.Linear calls of
 * RelPosAttention / AttnBlock, model.py:448-514, and the value heads,
 * model.py:990-1002):
 *   a = ln_w ? LayerNorm(x[r]) * ln_w + ln_b : x[r]       (x bf16, K = in)
 *   y = a @ W^T + bias                                      (fp32 acc)
 *   mode PLAIN: out = y (bf16)          mode GELU: out = gelu_erf(y)
 *   mode RESID: out[r] = resid[r] + gamma * (mask[r] ? y : 0)   (out may alias resid)
 *               with tok_lo set, the token rows (r % S < n_tokens) carry a low part:
 *               v = resid[r] + lo[r] + gamma * y, out[r] = bf16(v),
 *               lo[r] = bf16(v - out[r]), lo[r] = tok_lo[((r / S) * n_tokens +
 *               r % S) * out_features ..] (bf16; may alias its input)
 *   mode QKV:  y split into q/k/v, heads, stored to qkv (3, B, H, S, dpad)
 * Rows r = (b, s) over B positions x S rows; x, out, resid strides per row
 * are given in elements; mask is per (b, s) (seq mask) or NULL.
 * ---------------------------------------------------------------------- */
#define SHRIMP_LIN_PLAIN 0
#define SHRIMP_LIN_GELU 1
#define SHRIMP_LIN_RESID 2
#define SHRIMP_LIN_QKV 3

typedef struct {
  const void* x;
  int64_t x_sr;
  const void* w; /* packed, in x out */
  const float* bias;
  const float* ln_w; /* (in) or NULL */
  const float* ln_b;
  float eps;
  int32_t mode;
  const void* resid;
  int64_t r_sr;
  const float* gamma;
  const uint8_t* mask; /* (rows) or NULL */
  void* out;
  int64_t o_sr;
  int32_t rows, in_features, out_features;
  /* QKV mode (and S for the RESID mode's token rows) */
  int32_t B, S, H, dpad;
  /* RESID mode: low parts of the token rows (B, n_tokens, out_features) bf16, or NULL */
  void* tok_lo;
  int32_t n_tokens;
} shrimp_linear_args;

int shrimp_linear(const shrimp_linear_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Fused LayerNorm + q/k/v projection (RelPosAttention.forward q_proj /
 * k_proj / v_proj on AttnBlock's ln1, model.py:448-492, 508-514; replaces
 * shrimp_linear's QKV mode for C = 128):
 *   n = LN1(x[r]) ;  [q | k | v] = n @ Wqkv^T + bqkv   -> qkv (3, B, H, S, dpad)
 * with rows r = (b, s). The padding lanes d..dpad of qkv are not written.
 * shrimp_pack_attn_qkv folds LN1's affine into the weights (W diag(ln_w),
 * b + W ln_b) and writes MFMA fragments, the folded bias and the column sums
 * of the bf16 weights (used by shrimp_attn_fused) to `packed`
 * (shrimp_attn_qkv_pack_bytes(C) bytes; 0 = unsupported C). qkv_w is the
 * (3C, C) concatenation of q_proj / k_proj / v_proj weights (fp32), qkv_b
 * their biases; `scratch` holds 3C * C floats during packing.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* x; /* (rows, x_sr) bf16 */
  int64_t x_sr;
  void* qkv;     /* (3, B, H, S, dpad) bf16 */
  const void* packed;
  float eps;     /* LN1 epsilon */
  int32_t rows, B, S, H, C, dpad;
} shrimp_qkv_args;

size_t shrimp_attn_qkv_pack_bytes(int C);
int shrimp_pack_attn_qkv(const float* qkv_w, const float* qkv_b, const float* ln_w,
                         const float* ln_b, void* packed, void* scratch, int C, void* stream);
int shrimp_attn_qkv(const shrimp_qkv_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Fused attention-block tail (AttnBlock.forward after the attention core,
 * model.py:508-514; replaces the out_proj / fc1 / fc2 nn.Linear calls, LN2
 * and the two LayerScale residuals):
 *   s1  = seq + lo + g_attn * (mask ? x @ Wo^T + bo : 0)          (fp32)
 *   h   = bf16(gelu_erf(LN2(s1) @ W1^T + b1))
 *   v   = s1 + g_mlp * (mask ? h @ W2^T + b2 : 0)                (fp32)
 *   seq = bf16(v) (in place);  token rows: lo = bf16(v - seq)
 * x: attention output rows (bf16), seq: residual stream rows (bf16), both
 * with element row strides; mask: per-row live flag (rows with mask 0 are
 * not written: their update is 0). lo: the low part of a token row (row r
 * with r % S < n_tokens) at tok_lo[((r / S) * n_tokens + r % S) * C ..]
 * (bf16, read and written in place), 0 for cell rows and when tok_lo is NULL;
 * the summary tokens feed the value heads, so their residual stream is kept
 * to about 16 significant bits, as the reference's autocast serve keeps it in
 * fp32. C = 128, hidden = 256: the packed weights (160 KiB of fragments) fill
 * one workgroup's LDS.
 *
 * shrimp_pack_attn_mlp folds g_attn into Wo / bo, LN2's affine into W1 / b1
 * and g_mlp into W2 / b2, then writes MFMA fragments and the folded biases to
 * `packed` (shrimp_attn_mlp_pack_bytes bytes; 0 = unsupported shape).
 * `scratch` is a device buffer of C * hidden floats used during packing.
 * Weights are nn.Linear layouts (out, in), fp32.
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* out_w;  /* (C, C) */
  const float* out_b;  /* (C) */
  const float* g_attn; /* (C) LayerScale after attention */
  const float* ln_w;   /* (C) LN2 */
  const float* ln_b;   /* (C) */
  const float* fc1_w;  /* (hidden, C) */
  const float* fc1_b;  /* (hidden) */
  const float* fc2_w;  /* (C, hidden) */
  const float* fc2_b;  /* (C) */
  const float* g_mlp;  /* (C) LayerScale after the MLP */
  int32_t C, hidden;
} shrimp_mlp_weights;

typedef struct {
  const void* x;
  int64_t x_sr;
  void* seq;
  int64_t s_sr;
  const uint8_t* mask;  /* (rows) */
  const void* packed;   /* shrimp_pack_attn_mlp output */
  float eps;            /* LN2 epsilon */
  int32_t rows, C, hidden;
  void* tok_lo;         /* (B, n_tokens, C) bf16 low parts of the token rows, or NULL */
  int32_t S, n_tokens;  /* rows per position, token rows per position */
} shrimp_mlp_args;

size_t shrimp_attn_mlp_pack_bytes(int C, int hidden);
int shrimp_pack_attn_mlp(const shrimp_mlp_weights* w, void* packed, void* scratch, void* stream);
int shrimp_attn_mlp(const shrimp_mlp_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Fused relative-position-biased, key-masked attention (online softmax).
 *
 * Replaces shrimp::attn_pair (packages/shrimp/python/shrimp/_triton_attn.py:132-167)
 * and the materialized / flex bias paths of RelPosAttention (model.py:448-492,
 * build_attn_bias :718-760, _build_pair_u8 :762-792):
 *   score[i, j] = q_i . k_j / sqrt(d) + bias(i, j, h);  out_i = softmax_j(score) v
 *   keys j >= seq_lens[b] are skipped.
 * Bias sources:
 *   pair mode (pair != NULL):   bias = table2[pair[b, i, j], h], table2 (rows, H)
 *                               fp32; the reference's pad row (-3e4) masks keys.
 *   coords mode (pair == NULL): rows < n_tokens are tokens; for cells
 *       pos = (clamp(dq,-M,M)+M)*(2M+1) + clamp(dr,-M,M)+M with (dq,dr) =
 *       coords[key] - coords[query], bias = btab[pos, h];
 *       btab rows (2M+1)^2 .. +2 hold (cell q, token k), (token q, cell k),
 *       (token q, token k); keys whose mask is 0 get weight exactly 0.
 *   btab is produced by shrimp_attn_bias_table (with log2(e) folded in).
 *   xtab (optional, same source): the LUT re-indexed without clamping over
 *       |dq|, |dr| <= SHRIMP_ATTN_XD, fp16, head pair major
 *       [(H + 1) / 2][SHRIMP_ATTN_XP][2] (layout at shrimp_attn_bias_table);
 *       positions whose live cells span <= XD in q and r index it linearly.
 * q, k, v: (B, H, S, dpad) bf16 with head-dim zero padding; o element
 * (b, h, s, e) at o[b*o_sb + h*o_sh + s*o_sr + e], e < d (o_sh = d, o_sr = C
 * gives the (B, S, C) layout out_proj reads; o_sh = S*d, o_sr = d gives
 * (B, H, S, d)). Query rows >= seq_lens[b] store 0.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  int64_t qkv_sb, qkv_sh; /* elements between positions / heads; rows are dpad apart */
  const int32_t* seq_lens; /* (B) */
  /* pair mode */
  const uint8_t* pair;
  int64_t p_sb, p_sq;
  const float* table2; /* (table_rows, H) raw (log2e not folded) */
  int32_t table_rows;
  /* coords mode */
  const int32_t* coords; /* (B, S - n_tokens, 2) */
  const uint8_t* mask;   /* (B, S - n_tokens) */
  const float* btab;     /* ((2M+1)^2 + 3, H), log2e folded */
  const void* xtab;      /* ((H+1)/2, XP, 2) fp16, log2e folded, or NULL */
  int32_t lut_m, n_tokens;
  void* o;
  int64_t o_sb, o_sh, o_sr;
  int32_t B, S, H, d, dpad;
} shrimp_attn_args;

int shrimp_attn(const shrimp_attn_args* a, void* stream);

/* ------------------------------------------------------------------------
 * AttnBlock LN1 -> q/k/v projection -> attention in one launch
 * (model.py:497-503 then RelPosAttention, model.py:448-492): the result of
 * shrimp_attn_qkv followed by shrimp_attn up to rounding (LayerNorm is folded
 * into the projection, so the normalised rows are not rounded to bf16),
 * without the (3, B, H, S, dpad) q/k/v tensor. Each workgroup projects its
 * heads' keys and values into LDS and its queries into registers from the
 * position's rows and the packed weights of shrimp_pack_attn_qkv.
 * Covers C = 128, H = 8 (d = dpad = 16), coords mode, S <= 320; a->q, a->k,
 * a->v and a->qkv_* are not read. shrimp_attn_fused_supported(C, H, S,
 * dpad) is 1 for those shapes (other shapes take the two launches).
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* x;        /* (B, S, C) bf16 block input (before LN1) */
  int64_t x_sb, x_sr;   /* elements between positions / rows */
  const void* packed;   /* shrimp_pack_attn_qkv output */
  float eps;            /* LN1 epsilon */
} shrimp_attn_proj_args;

int shrimp_attn_fused_supported(int C, int H, int S, int dpad);
int shrimp_attn_fused(const shrimp_attn_args* a, const shrimp_attn_proj_args* p, void* stream);

/* ------------------------------------------------------------------------
 * Staged attention: the same operator as shrimp_attn in coords mode
 * (RelPosAttention, model.py:448-492; the serve kernel _triton_attn.py:59-130)
 * with its inputs in layouts the kernel copies into LDS by DMA.
 *   shrimp_attn_keys: once per forward, the key table of every position
 *     (classes, coordinates, LINEAR offset codes, per-16-key-block flags, the
 *     span test), shrimp_attn_keys_bytes(S) bytes per position, from the
 *     coords / mask / seq_lens that shrimp_attn reads (the per-block setup of
 *     model.py:718-760 done once for all heads and attention blocks).
 *   shrimp_attn_qkv_kvf: shrimp_attn_qkv (C = 128, H = 8, dpad = 16,
 *     S % 4 == 0) with q in the first plane of a->qkv ((B, H, S, 16)) and k,
 *     v in kvf as (B, H, 2, SP, 16) bf16 MFMA fragments, SP = S rounded up to
 *     16 (slots of keys >= S are not written and not read).
 *   shrimp_attn_staged: a->q, a->qkv_sb / qkv_sh the q layout above, kvf and
 *     meta from the two calls above, btab and xtab required, pair NULL;
 *     a->k, a->v, a->coords and a->mask are not read. With kvf NULL, K and V
 *     are the rows a->k, a->v in the layout of a->q ((B, H, S, 16) with the
 *     same strides, as shrimp_attn reads them; the operator path of config 2):
 *     the kernel permutes K into fragment order as it copies it and
 *     transposes V in LDS, with rows of dead keys (masked cells, keys past
 *     seq_lens) taken as zeros. Results equal
 *     shrimp_attn's up to the bf16 rounding of P (the softmax offsets may
 *     differ). shrimp_attn_staged_supported(H, S, dpad): dpad = 16, even H,
 *     S % 4 == 0, S <= 1024 and the workgroup's LDS within the device's
 *     per-workgroup limit: four waves while it fits 64 KiB (three workgroups
 *     per compute unit), eight waves with a compute unit's LDS past it
 *     (S >= 368, the spec-sized supports the evaluator pads to 384-576).
 * ---------------------------------------------------------------------- */
size_t shrimp_attn_keys_bytes(int S);
int shrimp_attn_keys(const int32_t* coords, const uint8_t* mask, const int32_t* seq_lens, int B,
                     int S, int n_tokens, int32_t* meta, void* stream);
/* shrimp_attn_keys and shrimp_fill_tokens(tokens, n_tokens, C, seq, seq_sb,
 * tok_lo, B) in one launch, with the same outputs and argument rules: the
 * forward writes its token rows and key table together (neither has a
 * counterpart in the reference; the token rows are model.py:905-926). */
int shrimp_attn_keys_tokens(const int32_t* coords, const uint8_t* mask, const int32_t* seq_lens,
                            int B, int S, int n_tokens, int32_t* meta, const float* tokens, int C,
                            void* seq, int64_t seq_sb, void* tok_lo, void* stream);
int shrimp_attn_qkv_kvf(const shrimp_qkv_args* a, void* kvf, void* stream);
int shrimp_attn_staged_supported(int H, int S, int dpad);
int shrimp_attn_staged(const shrimp_attn_args* a, const void* kvf, const int32_t* meta,
                       void* stream);

#define SHRIMP_ATTN_XD 26
/* offsets per head pair in xtab: (2 XD + 1)^2 = 2809 padded to 2816 (11 KiB of
 * dwords, which the staged kernel copies in whole 1 KiB DMAs) */
#define SHRIMP_ATTN_XP 2816

/* btab[pos, h] = log2(e) * table[lut[pos], h] for pos < (2M+1)^2 and the 3
 * token rows from table rows tok_rows[0..2]; table (rows, H) fp32.
 * xtab (if not NULL), ((H + 1) / 2) * SHRIMP_ATTN_XP * 2 fp16:
 * xtab[p, x, j] = fp16(btab[clamped pos of (dq, dr)], 2 p + j) with
 * x = (dq + XD) * (2 XD + 1) + dr + XD < (2 XD + 1)^2; zeros for the padding
 * x and for j = 1 of the last pair of an odd H. The two heads of a pair share
 * a dword per offset. */
int shrimp_attn_bias_table(const float* table, int table_rows, int H, const uint8_t* lut,
                           int lut_m, int tok_row_ct, int tok_row_tc, int tok_row_tt,
                           float* btab, void* xtab, void* stream);

/* ------------------------------------------------------------------------
 * Index preparation (model.py:861-863, 884-892, 905; batching.py:264-276):
 * one pass per position over the padded batch.
 *   nbr (B, N, 6) of dtype nbr_dt (i64 / i32 with sentinel N, or u16 with
 *   0xFFFF) -> idx (B, N, 7) int32, tap 0 = self, missing = N
 *   mask (B, N) bool/u8 -> mask8; coords (B, N, 2) i64/i32 -> coords32
 *   seq_lens[b] = n_tokens + (last live cell + 1)
 *   seq_mask (B, n_tokens + N) u8: 1 for token rows, mask for cell rows
 *   feats (B, N, F) of feats_dt -> xin (B, N, 32) bf16 zero-padded (if feats)
 * Any output pointer may be NULL to skip it.
 * ---------------------------------------------------------------------- */
int shrimp_prep_inputs(const void* nbr, int nbr_dt, const void* mask, const void* coords,
                       int coords_dt, const void* feats, int feats_dt, int nfeat, int B, int N,
                       int n_tokens, int32_t* idx, uint8_t* mask8, int32_t* coords32,
                       int32_t* seq_lens, uint8_t* seq_mask, void* xin, void* stream);

/* Serve pack + index preparation from the ABI-1 payload, on the device
 * (inference.py:865-892 _pack_group / serve_pack.rs:155-216 pack_group, then
 * the preparation above): rows row0 .. row0 + B - 1 of the CSR payload arrays
 *   node_feats (T, nfeat) f16, node_qr (T, 2) i16, nbr (T, 6) u16 (0xFFFF =
 *   absent; row-local indices), row_offsets (rows + 1) int64
 * padded to N cells, written as shrimp_prep_inputs writes them (idx, mask8,
 * coords32, seq_lens, seq_mask, xin; any output may be NULL). A row's live
 * cells are its first n = row_offsets[r + 1] - row_offsets[r] (clamped to N);
 * seq_lens = n_tokens + n. */
int shrimp_prep_csr(const void* node_feats, int nfeat, const int16_t* node_qr, const uint16_t* nbr,
                    const int64_t* row_offsets, int row0, int B, int N, int n_tokens, int32_t* idx,
                    uint8_t* mask8, int32_t* coords32, int32_t* seq_lens, uint8_t* seq_mask,
                    void* xin, void* stream);

/* seq[b, t, :] = bf16(tokens[t, :]) for t < n_tokens; seq rows are C apart,
 * positions seq_sb apart. tok_lo (optional, (B, n_tokens, C) bf16):
 * tok_lo[b, t, :] = bf16(tokens[t, :] - seq[b, t, :]), the low parts that the
 * residual kernels carry for the token rows. */
int shrimp_fill_tokens(const float* tokens, int n_tokens, int C, void* seq, int64_t seq_sb,
                       void* tok_lo, int B, void* stream);

/* ------------------------------------------------------------------------
 * Featurizer on the device (support.py:84-205 build_support, features.py:80-240
 * build_features with the window scan and the opponent's last turn; the
 * production featurizer is Rust, support.rs:52 / features.rs:19).
 * Position b owns the placement records [rec_offsets[b], rec_offsets[b+1]),
 * in placement order: cell rec_qr[i] = (q, r), owner rec_owner[i] (0 / 1),
 * placement index rec_index[i] (NULL: the record's ordinal). player and
 * phase (0 opening, 1 first stone, 2 second stone) may be NULL: they are then
 * derived from the record count as for a decision state (player 0 opens,
 * then two stones per turn), and in phase 2 the last record is the turn's
 * first stone. Support radius R (1..24): legal = empty cells within R of a
 * stone, halo = distance R + 1; hot / win-now cells from the single-colour
 * length-6 window scan. Outputs, Npad rows per position (collate layout,
 * batching.py:45-80):
 *   feats (B, Npad, 15) f32, nbr (B, Npad, 6) int32 row-local (absent and
 *   padding rows = Npad), mask (B, Npad) u8, coords (B, Npad, 2) int32;
 *   counts (B, 4) int32 = nodes, legal, stones, halo;
 *   status (B) int32: 0 ok, 2 the support does not fit the 64 x 64 cell
 *   window of one workgroup (outputs zero), 3 more nodes than Npad (rows past
 *   Npad dropped).
 * feats == NULL computes counts and status only (to choose Npad).
 * ---------------------------------------------------------------------- */
int shrimp_featurize(const int32_t* rec_qr, const uint8_t* rec_owner, const int32_t* rec_index,
                     const int64_t* rec_offsets, const uint8_t* player, const uint8_t* phase,
                     int B, int radius, int Npad, float* feats, int32_t* nbr, uint8_t* mask,
                     int32_t* coords, int32_t* counts, int32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Trunk tail + value head (model.py:927-935, 990-1002):
 *   seq_f = LayerNorm(seq) (all S rows, fp32 stats), cell rows * mask -> out_seq (bf16);
 *           token rows are seq + tok_lo when tok_lo is set (bf16 seq only)
 *   pooled = masked mean of the normalized cells (count clamped to 1)
 *   value = value_head(relu(value_reduction([T0, T1, pooled])))  -> value (B, 65) fp32
 *   moves_left likewise from [T4, T5, pooled] when moves_left is non-NULL.
 * Head weights are fp32 and TRANSPOSED relative to nn.Linear.weight:
 *   vr_w / mr_w (3C, C) = reduction.weight^T, vh_w / mh_w (C, bins) = head.weight^T.
 * workspace: caller-provided (B, 6C) fp32 scratch (the head inputs).
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* seq; /* (B, S, C) bf16 */
  int64_t s_sb;
  const uint8_t* mask; /* (B, N) */
  const float* ln_w;
  const float* ln_b;
  float eps;
  void* out_seq; /* (B, S, C) bf16 */
  const float* vr_w; const float* vr_b; /* (3C, C)^T layout, (C) */
  const float* vh_w; const float* vh_b; /* (C, bins)^T layout, (bins) */
  float* value;                         /* (B, bins) */
  const float* mr_w; const float* mr_b;
  const float* mh_w; const float* mh_b;
  float* moves_left;
  float* workspace; /* (B, 6C) */
  int32_t B, S, n_tokens, C, bins;
  const void* tok_lo; /* (B, n_tokens, C) bf16 low parts of the token rows, or NULL */
} shrimp_tail_args;

int shrimp_trunk_tail(const shrimp_tail_args* a, void* stream);

/* Trunk tail and policy head in one pass over the cells (model.py:927-935,
 * 990-1020; no single counterpart in the reference, which normalises, pools
 * and runs the policy head as separate modules): shrimp_trunk_tail(tail)
 * followed by shrimp_hex_conv(policy) on tail's normalised cell rows, with the
 * same results, except that the normalised rows stay in the policy conv's
 * workgroup: tail->out_seq is not written. tail: as for shrimp_trunk_tail,
 * bf16 seq with C = 128 and 16-byte aligned rows. policy: the 7-tap
 * 128 -> 128 conv + bias + ReLU + Linear(C, 1) head (w, bias, head_w, head_b,
 * head_out, relu = 1, idx, idx_stride, B, N = S - n_tokens) reading the cell
 * rows of tail->seq: x = seq + n_tokens * 128, x_sb = tail->s_sb, x_sn = 128,
 * mask = tail->mask. shrimp_policy_tail_supported reports whether the fused
 * kernel covers N cells of C channels (else SHRIMP_EINVAL). */
int shrimp_policy_tail_supported(int N, int C);
int shrimp_policy_tail(const shrimp_conv_args* policy, const shrimp_tail_args* tail, void* stream);

/* shrimp_trunk_tail without a workspace: no counterpart in the reference. It
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serve loops, harnesses that forbid hipMalloc). The head
 * inputs live in a fixed device array of SHRIMP_TAIL_SCRATCH_FLOATS floats
 * (8 MiB) that the library holds on each device it runs on until the process
 * ends; a->workspace is ignored. Requires B * 6 * C <= SHRIMP_TAIL_SCRATCH_FLOATS
 * (else SHRIMP_EINVAL, nothing launched). Calls on one device share that
 * array: calls that overlap in time on one device (other streams, other host
 * threads) race and must be serialised by the caller. Allocates nothing. */
#define SHRIMP_TAIL_SCRATCH_FLOATS (2 * 1024 * 1024)
int shrimp_trunk_tail_noalloc(const shrimp_tail_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Serve decode (inference.py:998-1042, losses.py:40-60):
 *   value[b] = clamp(sum softmax(value_logits[b]) * linspace(-1,1,bins), -1, 1)
 *   ml[b]    = (clamp(...) + 1) / 2 * ml_cap                  (if ml_logits)
 *   priors[out_off[b] + i] = softmax(policy[b, :legal[b]])_i  (fp32)
 *     (policy rows are pol_sb apart and pol_sb long; legal[b] is clamped to it)
 *   logits_out[out_off[b] + i] = policy[b, i]                  (if logits_out)
 * ---------------------------------------------------------------------- */
int shrimp_decode(const float* value_logits, const float* ml_logits, const float* policy,
                  int64_t pol_sb, const int32_t* legal, const int64_t* out_off, int B, int bins,
                  float ml_cap, float* value, float* ml, float* priors, float* logits_out,
                  void* stream);

/* ------------------------------------------------------------------------
 * Index builders kept for the reference operator ABI and its tests.
 *   pair (B, S, S) u8 (model.py:762-792): rows from the (2M+1)^2 LUT for
 *     cell pairs (key - query offset), token rows, pad keys -> pad_row.
 *   ray gather index (B, N, 32) int32 (hexfield_eq/_triton_ray.py:221-281):
 *     slot 0 = self, slot 1 + axis*10 + dir*5 + (k-1) = live cell at
 *     coords + dir_sign * k * axis (axes Q, R, QR), slot 31 = N.
 * ---------------------------------------------------------------------- */
int shrimp_build_pair_u8(const int32_t* coords, const uint8_t* mask, const uint8_t* lut,
                         int lut_m, int B, int N, int n_tokens, int row_ct, int row_tc,
                         int row_tt, int pad_row, uint8_t* pair, void* stream);
int shrimp_build_ray_index(const int32_t* coords, const uint8_t* mask, int B, int N,
                           int32_t* idx, void* stream);

/* ------------------------------------------------------------------------
 * hexfield_eq::ray_attn (hexfield_eq/_triton_ray.py:681-715; kernel :378-501):
 * gathered ray attention over the 32-slot index above.
 *   q, k, v, out: (B, H, N, D) fp16, D in {16, 32, 64, 128}, element strides
 *     *_sb / *_sh / *_sn (multiples of 8 in [0, 2^31), bases 16-byte aligned;
 *     the head dimension is contiguous; a head pair's rows of a position span
 *     less than 2 GiB). The (B, N, H, D).transpose(1, 2) views the reference
 *     passes satisfy this.
 *   idx (B, N, 32) int32, strides idx_sb / idx_sn, slot stride 1; an entry
 *     outside [0, N) is an absent key.
 *   slot_bias (32, H) fp16 (the reference rounds its fp32 slot bias to fp16).
 *   raylen (B, N, 12) u8, strides rl_sb / rl_sn; read only when blockers != 0
 *     (may be NULL otherwise).
 *   seq_lens (B,) int32: rows >= seq_lens[b] are written as zeros.
 * Head h rides win axis h / 2 and side h % 2: slot s of row i is live when
 * idx[i, s] is present and s == 0, or s = 1 + (h/2)*10 + dir*5 + (k-1) with
 * k <= raylen[i, (h%2)*6 + (h/2)*2 + dir] (k <= 5 without blockers); heads
 * h >= 6 see only slot 0.
 *   out = sum_s softmax(q . k_s / sqrt(D) + slot_bias[s, h]) v_s (fp32 math,
 *   fp16 store); a row without a live slot is zero.
 * ---------------------------------------------------------------------- */
typedef struct {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_sb, q_sh, q_sn;
  int64_t k_sb, k_sh, k_sn;
  int64_t v_sb, v_sh, v_sn;
  const int32_t* idx;
  int64_t idx_sb, idx_sn;
  const uint16_t* slot_bias;
  const uint8_t* raylen;
  int64_t rl_sb, rl_sn;
  const int32_t* seq_lens;
  uint16_t* out;
  int64_t o_sb, o_sh, o_sn;
  int B, H, N, D;
  int blockers;
} shrimp_ray_attn_args;

int shrimp_ray_attn(const shrimp_ray_attn_args* a, void* stream);
/* Kernel selection for tests and measurement: 0 = automatic (the head pair's
 * K/V rows staged in LDS when 8 * N * D <= 64 KiB, else gathered from global
 * memory), 1 = always global. Returns the previous setting. */
int shrimp_ray_attn_variant(int v);

/* ------------------------------------------------------------------------
 * hexfield_eq::hex_conv_ln_raytap, K1 (hexfield_eq/_triton_conv.py:501-555;
 * kernel :391-499): ray-tap conv + LayerNorm (+ReLU) + row mask.
 *   x (B, N, C) fp16, strides x_sb / x_sn (multiples of 8, 16-byte aligned).
 *   gather_idx (B, N, >= 1) int32, strides g_sb / g_sn: tap 0 (the centre row)
 *     is the only tap read; an entry outside [0, N) reads a zero row.
 *   ray_idx (B, N, 32) int32 and reach (B, N, 2, 6) u8 ([side][tap - 1]),
 *     strides r_sb / r_sn and re_sb / re_sn.
 *   alpha (5, C) fp16; corb the orbit width (C % corb == 0, corb % 8 == 0):
 *     channel c is on side (c % corb) >= corb / 2.
 *   tap t = 1..6, channel c: sum_{k=1..5} alpha[k-1, c] * x[ray_idx[i,
 *     slot(t, k)], c] over the k <= reach[i, side(c), t-1] with a present
 *     index (fp32 sum, stored as fp16), slot(t, k) = 1 + axis*10 + dir*5 +
 *     (k-1) for the tap's (axis, dir).
 *   conv = [x[centre] | tap 1 .. tap 6] . W + bias, W (7C, Cout) fp16 packed by
 *     shrimp_pack_raytap_weight, fp32 accumulation; y = LayerNorm(conv) over
 *     Cout with ln_w / ln_b (fp32, eps); ReLU if relu; rows with mask 0 -> 0;
 *     out (B, N, Cout) fp16, 16-byte aligned, strides o_sb / o_sn (multiples of 8).
 *   mask (B, N) u8, row stride N.
 * C and Cout in {64, 96, 128}; N <= 512.
 * ---------------------------------------------------------------------- */
typedef struct {
  const uint16_t* x;
  int64_t x_sb, x_sn;
  const int32_t* gather_idx;
  int64_t g_sb, g_sn;
  const uint8_t* mask;
  const void* packed_w;
  const float* bias;
  const float* ln_w;
  const float* ln_b;
  const int32_t* ray_idx;
  int64_t r_sb, r_sn;
  const uint8_t* reach;
  int64_t re_sb, re_sn;
  const uint16_t* alpha;
  float eps;
  int relu;
  int corb;
  uint16_t* out;
  int64_t o_sb, o_sn;
  int B, N, C, Cout;
} shrimp_raytap_args;

/* Bytes of the packed K1 weight for (C, Cout); 0 if unsupported. */
size_t shrimp_raytap_wpack_bytes(int C, int Cout);
/* w (7, C, Cout) fp16 row-major (= the reference's weight.reshape(7C, Cout))
 * -> packed fp16 MFMA fragments. */
int shrimp_pack_raytap_weight(const uint16_t* w, int C, int Cout, void* packed, void* stream);
int shrimp_conv_ln_raytap(const shrimp_raytap_args* a, void* stream);

/* ------------------------------------------------------------------------
 * fp32 serve mode: the forward with fp32 activations end to end, as the
 * reference serves with autocast off (SHRIMP_SERVE_AUTOCAST=0,
 * packages/shrimp/python/shrimp/inference.py:50-68; model.py:346-514 run in
 * fp32). Same argument structs and semantics as the bf16 entry points above,
 * with these differences:
 *   - activations (x, resid, out, seq, out_seq, q, k, v, o) are fp32;
 *   - weights are packed by the *_f32 packers into 4 bytes per weight, in
 *     one of two layouts chosen by the per-tap input width kin (cin_pad for
 *     conv weights, tap-major; in_features for linear weights). kin a
 *     multiple of 32: per tap, k-chunk kc (32 rows) and output block nb (16
 *     outputs) a 1 KiB hi fragment then a 1 KiB lo fragment, lane l holding
 *     8 bf16 of W[32 kc + 8 (l / 16) + e][16 nb + l % 16] (hi = bf16(w), lo =
 *     bf16(w - hi)); the GEMMs then run on bf16 MFMA with x split the same
 *     way, three products per tile (hi·lo + lo·hi + hi·hi, fp32
 *     accumulation). Otherwise (kin 16): per tap, kc (16 rows) and nb,
 *     16-byte fp32 fragments, lane l holding W[16 kc + 4 (l / 16) + j][16 nb
 *     + l % 16], j < 4, for fp32 MFMA;
 *   - shrimp_hex_conv_f32: cin_pad and cout multiples of 16; LayerNorm and
 *     head epilogues need cout in {32, 64, 96, 128, 192, 256};
 *   - shrimp_linear_f32: in / out features multiples of 16; QKV mode writes
 *     (3, B, H, S, dpad) fp32 with dpad >= d, dpad % 4 == 0;
 *   - shrimp_attn_f32: q, k, v (B, H, S, dpad) fp32, d <= 64, any S; pair or
 *     coords bias as shrimp_attn (btab and table2 fp32; xtab unused). At
 *     d = dpad = 16 in coords mode (lut_m <= 26, 16-byte aligned q/k/v/o,
 *     strides multiples of 4, the sequence within one workgroup's LDS) it runs
 *     on bf16 MFMA with each fp32 operand split into hi and lo bf16 parts
 *     (three products per tile, fp32 accumulation and softmax); otherwise,
 *     and at attention variant 3, one query row per thread with keys streamed
 *     through LDS;
 *   - shrimp_trunk_tail_f32: seq and out_seq fp32;
 *   - shrimp_prep_feats_f32 / shrimp_prep_csr_feats_f32: the stem input
 *     xin (B, N, 16) fp32 (features zero-padded to 16 channels) from padded
 *     feats of feats_dt (nfeat <= 16) or from the ABI-1 CSR f16 node_feats
 *     (rows as in shrimp_prep_csr); the other preparation outputs come from
 *     shrimp_prep_inputs / shrimp_prep_csr with xin = NULL;
 *   - shrimp_fill_tokens_f32: token rows of an fp32 seq.
 * ---------------------------------------------------------------------- */
size_t shrimp_conv_wpack_bytes_f32(int taps, int cin_pad, int cout);
int shrimp_pack_conv_weight_f32(const float* w, float* packed, int taps, int cin, int cin_pad,
                                int cout, void* stream);
int shrimp_pack_linear_weight_f32(const float* w, float* packed, int in_features,
                                  int out_features, void* stream);
int shrimp_hex_conv_f32(const shrimp_conv_args* a, void* stream);
int shrimp_linear_f32(const shrimp_linear_args* a, void* stream);
int shrimp_attn_f32(const shrimp_attn_args* a, void* stream);
int shrimp_trunk_tail_f32(const shrimp_tail_args* a, void* stream);
int shrimp_prep_feats_f32(const void* feats, int feats_dt, int nfeat, int B, int N, float* xin,
                          void* stream);
int shrimp_prep_csr_feats_f32(const void* node_feats, int nfeat, const int64_t* row_offsets,
                              int row0, int B, int N, float* xin, void* stream);
int shrimp_fill_tokens_f32(const float* tokens, int n_tokens, int C, float* seq, int64_t seq_sb,
                           int B, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SHRIMP_HIP_H */
