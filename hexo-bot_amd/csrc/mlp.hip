// Fused tail of the attention block for gfx950 (AttnBlock.forward after the
// attention core, packages/shrimp/python/shrimp/model.py:508-514):
//
//   s1  = seq + g_attn * (m * (att . Wo^T + bo))          (out_proj, LayerScale)
//   h   = GELU_erf(LN2(s1) . W1^T + b1)                   (fc1, hidden 2C)
//   seq = s1 + g_mlp * (m * (h . W2^T + b2))              (fc2, LayerScale)
// s1 stays in fp32 inside the kernel: it is the fc2 accumulators' starting
// value, so only the block's result is rounded to bf16. The summary-token
// rows carry the rounding remainder as a second bf16 (tok_lo), so their
// residual stream keeps about 16 significant bits across the blocks (the
// reference's autocast serve keeps the stream in fp32; the tokens feed the
// value heads).
//
// The per-channel factors are folded into the weights once, at pack time
// (shrimp_pack_attn_mlp):
//   Wo' = diag(g_attn) Wo,  bo' = g_attn * bo
//   W1' = W1 diag(ln_w),    b1' = b1 + W1 ln_b
//   W2' = diag(g_mlp) W2,   b2' = g_mlp * b2
// so per row the kernel computes
//   s1 = seq + lo + (att . Wo'^T + bo'),  n = (s1 - mean) * rstd,
//   h = GELU(n . W1'^T + b1'),            v = (s1 + b2') + h . W2'^T,
//   seq = bf16(v), token rows: lo = bf16(v - seq)
// with n and h in bf16 as MFMA inputs. Rows with m = 0 are left untouched
// (their updates are multiplied by 0), so the math runs unmasked and only
// live rows store.
//
// Layout: one persistent workgroup per CU keeps the packed fragments of the
// three matrices in LDS (C = 128: 32 + 64 + 64 KiB = the whole 160 KiB); each
// of its 16 waves (four per SIMD, at most 128 VGPRs each: the rows are not
// requested a block ahead, the other waves of the SIMD cover their latency)
// streams blocks of 16 rows through the three products without leaving
// registers: a product's output fragment (lane l: channels
// 16 nb + 4 (l/16) + j of row l % 16) is directly the next product's input
// fragment for K-step nb / 2, because W1' and W2' are packed with that
// interleaved K order. The biases enter as the accumulators' initial values.
// Only att and seq touch HBM: 3 x 256 bytes per row.
#include <algorithm>

#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

// Weight fragment packer shared with the conv / linear packers (hex_conv.hip).
__global__ void pack_weight_kernel(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                   int K, int NOUT, int cin, int cin_pad, int64_t s_t,
                                   int64_t s_c, int64_t s_n, int interleaved);

namespace {

constexpr int MC = 128;           // channels
constexpr int MH = 2 * MC;        // hidden width
constexpr int MWAVES = 16;        // waves per workgroup (4 per SIMD)
constexpr uint32_t WO_OFF = 0;                        // out_proj fragments
constexpr uint32_t W1_OFF = MC * MC * 2;              // fc1 fragments
constexpr uint32_t W2_OFF = W1_OFF + MC * MH * 2;     // fc2 fragments
constexpr uint32_t W_LDS = W2_OFF + MH * MC * 2;      // 163840 bytes
constexpr uint32_t BO_OFF = W_LDS;                    // folded biases (fp32) after the fragments
constexpr uint32_t B1_OFF = BO_OFF + MC * 4;
constexpr uint32_t B2_OFF = B1_OFF + MH * 4;
constexpr uint32_t PACK_BYTES = B2_OFF + MC * 4;

// GELU(x) = x Phi(x) = max(x, 0) - |x| h(|x|), h(a) = erfc(a / sqrt(2)) / 2.
// h is evaluated as exp2(-g(a)) with g a degree-5 polynomial fitted (weighted
// least squares on a in [0, 5], weight a h(a)) to -log2 h(a), and a clamped at
// 5 (h(5) = 2.9e-7): one transcendental and seven fused multiply-adds per
// value. Against float64 erf-GELU the error is at most 3.8e-6 absolute over
// [-12, 12] (a tenth of a bf16 rounding step of the output near 0.1), and the
// kernel rounds the result to bf16 for fc2. The clamp is one med3 and max(x, 0)
// one integer max (relu_bits): fminf / fmaxf on an MFMA result cost a second
// instruction each, a canonicalisation of the operand the compiler cannot
// prove canonical.
SHRIMP_DEV float gelu_ex2(float x) {
  constexpr float g0 = 1.0001733303070068f, g1 = 1.149885654449463f, g2 = 0.461910218000412f;
  constexpr float g3 = 0.05010765790939331f, g4 = -0.006412093993276358f;
  constexpr float g5 = 0.00037955178413540125f;
  const float ax = fabsf(x);
  const float a = __builtin_amdgcn_fmed3f(ax, 0.0f, 5.0f);
  float g = fmaf(g5, a, g4);
  g = fmaf(g, a, g3);
  g = fmaf(g, a, g2);
  g = fmaf(g, a, g1);
  g = fmaf(g, a, g0);
  const float h = __builtin_amdgcn_exp2f(-g);
  return fmaf(-ax, h, relu_bits(x));
}

SHRIMP_DEV u32x4 lds_frag(const unsigned char* wl, uint32_t base, int ks, int nb, int nbt,
                          int lane) {
  return *reinterpret_cast<const u32x4*>(wl + base + (uint32_t)(((ks * nbt + nb) * 64 + lane) * 16));
}

// The folded biases [bo' | b1' | b2'] are 32 blocks of 16 channels, kept in
// registers (BiasRegs): the loop body issues no bias loads.
typedef BiasRegs<(MC + MH + MC) / 16> MlpBias;

// Attention-output fragments (out_proj input) of one 16-row block; rows at
// or past `rows` read as zeros.
SHRIMP_DEV void load_x(const shrimp_mlp_args& a, __amdgpu_buffer_rsrc_t xr, int row, int lg,
                       u32x4 (&xf)[MC / 32]) {
  const uint32_t xo =
      row < a.rows ? (uint32_t)((int64_t)row * a.x_sr * 2) + (uint32_t)(lg * 16) : SHRIMP_OOB_OFFSET;
#pragma unroll
  for (int ks = 0; ks < MC / 32; ++ks) xf[ks] = buf_load16(xr, xo + ks * 64);
}

// Residual rows (bf16, this lane's 4-channel groups) of the row `row`; rows at
// or past `rows` read as zeros.
SHRIMP_DEV void load_s(const shrimp_mlp_args& a, __amdgpu_buffer_rsrc_t sr, int row, int lg,
                       u32x2 (&sf)[MC / 16]) {
  const uint32_t so =
      row < a.rows ? (uint32_t)((int64_t)row * a.s_sr * 2) + (uint32_t)(lg * 8) : SHRIMP_OOB_OFFSET;
#pragma unroll
  for (int nb = 0; nb < MC / 16; ++nb) sf[nb] = buf_load8(sr, so + nb * 32);
}

// One block of 16 rows (lane: row lane % 16, channel group lane / 16); xf:
// the block's attention-output fragments; loff: this lane's byte offset in
// the token low parts (lor), past the resource for cell rows.
SHRIMP_DEV void mlp_block(const shrimp_mlp_args& a, const unsigned char* wl, const MlpBias& bias,
                          __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t lor, uint32_t loff,
                          const u32x4 (&xf)[MC / 32], int row, int lane, bool store) {
  constexpr int KS1 = MC / 32, NB1 = MC / 16, NBH = MH / 16, KT = MH / 32, NB2 = MC / 16;
  constexpr int TB1 = NB1, TB2 = NB1 + NBH;  // first bias block of b1', b2'
  const int lg = lane >> 4;
  // the block's residual rows and their low parts (zeros for cells), consumed
  // after out_proj
  u32x2 sin[MC / 16], slo[MC / 16];
  load_s(a, sr, row, lg, sin);
#pragma unroll
  for (int nb = 0; nb < NB1; ++nb) slo[nb] = buf_load8(lor, loff + nb * 32);

  // accumulators start at the biases
  f32x4 acc[NB1];
#pragma unroll
  for (int nb = 0; nb < NB1; ++nb) acc[nb] = bias.rows(nb);

  // ---- out_proj ----------------------------------------------------------
  // (scheduling barriers keep the weight-fragment reads next to their MFMAs;
  // hoisted all at once they would not fit in registers)
#pragma unroll
  for (int nb = 0; nb < NB1; ++nb) {
    u32x4 w[KS1];
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) w[ks] = lds_frag(wl, WO_OFF, ks, nb, NB1, lane);
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) acc[nb] = mfma16x16x32(w[ks], xf[ks], acc[nb]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- residual 1, LayerNorm 2 (affine folded into W1', b1') ---------------
  // s1 (fp32) is the fc2 accumulators' starting value, added to b2'.
  f32x4 acc2[NB2];
  float v[NB1][4];
#pragma unroll
  for (int nb = 0; nb < NB1; ++nb) {
    v[nb][0] = acc[nb][0] + (bf16_lo(sin[nb].x) + bf16_lo(slo[nb].x));
    v[nb][1] = acc[nb][1] + (bf16_hi(sin[nb].x) + bf16_hi(slo[nb].x));
    v[nb][2] = acc[nb][2] + (bf16_lo(sin[nb].y) + bf16_lo(slo[nb].y));
    v[nb][3] = acc[nb][3] + (bf16_hi(sin[nb].y) + bf16_hi(slo[nb].y));
    const f32x4 b2 = bias.rows(TB2 + nb);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc2[nb][j] = b2[j] + v[nb][j];
  }
  // one pass for the row statistics: four independent sum / sum-of-squares
  // chains, var = E[v^2] - mean^2, then one FMA per value
  float sj[4], qj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sj[j] = v[0][j];
    qj[j] = v[0][j] * v[0][j];
  }
#pragma unroll
  for (int nb = 1; nb < NB1; ++nb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sj[j] += v[nb][j];
      qj[j] = fmaf(v[nb][j], v[nb][j], qj[j]);
    }
  const float mean = sum_groups_swap((sj[0] + sj[1]) + (sj[2] + sj[3])) * (1.0f / MC);
  const float ex2 = sum_groups_swap((qj[0] + qj[1]) + (qj[2] + qj[3])) * (1.0f / MC);
  const float rstd = rsqrtf(fmaxf(fmaf(-mean, mean, ex2), 0.f) + a.eps);
  const float nmr = -mean * rstd;
  u32x4 hf[KS1];
#pragma unroll
  for (int ks = 0; ks < KS1; ++ks) {
    const int n0 = 2 * ks, n1 = 2 * ks + 1;
    hf[ks] = u32x4{pack_bf16x2(fmaf(v[n0][0], rstd, nmr), fmaf(v[n0][1], rstd, nmr)),
                   pack_bf16x2(fmaf(v[n0][2], rstd, nmr), fmaf(v[n0][3], rstd, nmr)),
                   pack_bf16x2(fmaf(v[n1][0], rstd, nmr), fmaf(v[n1][1], rstd, nmr)),
                   pack_bf16x2(fmaf(v[n1][2], rstd, nmr), fmaf(v[n1][3], rstd, nmr))};
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- fc1 -> GELU -> fc2, one 32-wide hidden slice at a time ---------------
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    f32x4 ah[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      u32x4 w[KS1];
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) w[ks] = lds_frag(wl, W1_OFF, ks, 2 * kt + hh, NBH, lane);
      ah[hh] = bias.rows(TB1 + 2 * kt + hh);
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) ah[hh] = mfma16x16x32(w[ks], hf[ks], ah[hh]);
    }
    // fc2 fragments in two halves, the first half's LDS reads overlapping the
    // GELU
    u32x4 w2[NB2 / 2];
#pragma unroll
    for (int nb = 0; nb < NB2 / 2; ++nb) w2[nb] = lds_frag(wl, W2_OFF, kt, nb, NB2, lane);
    u32x4 gf;
    gf[0] = pack_bf16x2(gelu_ex2(ah[0][0]), gelu_ex2(ah[0][1]));
    gf[1] = pack_bf16x2(gelu_ex2(ah[0][2]), gelu_ex2(ah[0][3]));
    gf[2] = pack_bf16x2(gelu_ex2(ah[1][0]), gelu_ex2(ah[1][1]));
    gf[3] = pack_bf16x2(gelu_ex2(ah[1][2]), gelu_ex2(ah[1][3]));
#pragma unroll
    for (int nb = 0; nb < NB2 / 2; ++nb) acc2[nb] = mfma16x16x32(w2[nb], gf, acc2[nb]);
#pragma unroll
    for (int nb = 0; nb < NB2 / 2; ++nb) w2[nb] = lds_frag(wl, W2_OFF, kt, NB2 / 2 + nb, NB2, lane);
#pragma unroll
    for (int nb = 0; nb < NB2 / 2; ++nb)
      acc2[NB2 / 2 + nb] = mfma16x16x32(w2[nb], gf, acc2[NB2 / 2 + nb]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- residual 2 -> seq (and the token rows' low parts) ----------------------
  if (store) {
    unsigned short* op = static_cast<unsigned short*>(a.seq) + (int64_t)row * a.s_sr + lg * 4;
#pragma unroll
    for (int nb = 0; nb < NB2; ++nb) {
      u32x2 pk, lo;
      pk.x = pack_bf16x2(acc2[nb][0], acc2[nb][1]);
      pk.y = pack_bf16x2(acc2[nb][2], acc2[nb][3]);
      lo.x = pack_bf16x2(acc2[nb][0] - bf16_lo(pk.x), acc2[nb][1] - bf16_hi(pk.x));
      lo.y = pack_bf16x2(acc2[nb][2] - bf16_lo(pk.y), acc2[nb][3] - bf16_hi(pk.y));
      *reinterpret_cast<u32x2*>(op + nb * 16) = pk;
      __builtin_amdgcn_raw_buffer_store_b64(lo, lor, loff + nb * 32, 0, 0);
    }
  }
}

}  // namespace

__global__ __launch_bounds__(MWAVES * 64, 1) void attn_mlp_kernel(const shrimp_mlp_args a,
                                                                  uint32_t x_bytes,
                                                                  uint32_t s_bytes,
                                                                  uint32_t lo_bytes) {
  extern __shared__ __attribute__((aligned(16))) unsigned char wl[];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();

  // The packed fragments of all three matrices into LDS (16-byte chunks).
  {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.packed, W_LDS);
    constexpr int CHUNKS = W_LDS / 16;
    constexpr int PER = (CHUNKS + MWAVES * 64 - 1) / (MWAVES * 64);
    u32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = buf_load16(wr, (uint32_t)(i * MWAVES * 64 + threadIdx.x) * 16);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t off = (uint32_t)(i * MWAVES * 64 + threadIdx.x) * 16;
      if (off < W_LDS) *reinterpret_cast<u32x4*>(wl + off) = v[i];
    }
  }
  __syncthreads();

  MlpBias bias;
  bias.load(reinterpret_cast<const float*>(static_cast<const unsigned char*>(a.packed) + BO_OFF),
            lane);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.seq, s_bytes);
  // token low parts: lo_bytes is 0 without them (every access reads zeros /
  // is dropped)
  const __amdgpu_buffer_rsrc_t lor = make_rsrc(a.tok_lo, lo_bytes);
  // row mask bytes: rows at or past `rows` read as 0 (not stored)
  const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.mask, (uint32_t)a.rows);
  // Contiguous, balanced range of 16-row blocks per wave; the next block's
  // mask byte is requested before the current block's math.
  const int64_t nblk = (a.rows + 15) / 16;
  const int64_t tw = (int64_t)gridDim.x * MWAVES;
  const int64_t gw = (int64_t)blockIdx.x * MWAVES + wave;
  const int begin = (int)(gw * nblk / tw);
  const int end = (int)((gw + 1) * nblk / tw);
  const int lr = lane & 15, lg = lane >> 4;
  auto load_m = [&](int row) {
    const uint32_t off = row < a.rows ? (uint32_t)row : SHRIMP_OOB_OFFSET;
    return (unsigned)__builtin_amdgcn_raw_buffer_load_b8(mr, off, 0, 0);
  };
  u32x4 cur[MC / 32];
  unsigned mcur = 0, mnxt = 0;
  if (begin < end) mnxt = load_m(begin * 16 + lr);
  for (int blk = begin; blk < end; ++blk) {
    mcur = mnxt;
    // past this wave's range: an offset past the resource (reads zero)
    const int nrow = blk + 1 < end ? (blk + 1) * 16 + lr : a.rows;
    // the next block's mask byte ahead of this block's rows: a wait for it
    // never waits for them
    mnxt = load_m(nrow);
    const int row = blk * 16 + lr;
    const int pos = row / a.S, srow = row - pos * a.S;
    const uint32_t loff = row < a.rows && srow < a.n_tokens
                              ? (uint32_t)(((pos * a.n_tokens + srow) * MC + lg * 4) * 2)
                              : SHRIMP_OOB_OFFSET;
    load_x(a, xr, row, lg, cur);
    mlp_block(a, wl, bias, sr, lor, loff, cur, row, lane, mcur != 0);
  }
}

// ---- packing: fold the per-channel factors, then fragment order -----------
__global__ void attn_mlp_bias_kernel(const shrimp_mlp_weights w, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < MC) {
    out[i] = w.g_attn[i] * w.out_b[i];                                  // bo'
  } else if (i < MC + MH) {
    const int n = i - MC;
    float s = w.fc1_b[n];
    for (int k = 0; k < MC; ++k) s = fmaf(w.fc1_w[(int64_t)n * MC + k], w.ln_b[k], s);
    out[i] = s;                                                         // b1'
  } else if (i < MC + MH + MC) {
    const int n = i - MC - MH;
    out[i] = w.g_mlp[n] * w.fc2_b[n];                                   // b2'
  }
}

// scaled[n][k] = rs[n] * src[n][k] * cs[k] (rs / cs may be NULL = 1)
__global__ void scale_rows_cols_kernel(const float* __restrict__ src, const float* __restrict__ rs,
                                       const float* __restrict__ cs, int n_out, int n_in,
                                       float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)n_out * n_in) return;
  const int n = (int)(i / n_in), k = (int)(i - (int64_t)n * n_in);
  float v = src[i];
  if (rs) v *= rs[n];
  if (cs) v *= cs[k];
  dst[i] = v;
}

}  // namespace shrimp

using namespace shrimp;

extern "C" size_t shrimp_attn_mlp_pack_bytes(int C, int hidden) {
  return (C == MC && hidden == MH) ? (size_t)PACK_BYTES : 0;
}

extern "C" int shrimp_pack_attn_mlp(const shrimp_mlp_weights* w, void* packed, void* scratch,
                                    void* stream) {
  SHRIMP_REQUIRE(w && packed && scratch, "pack_attn_mlp: null pointer");
  SHRIMP_REQUIRE(w->C == MC && w->hidden == MH,
                 "pack_attn_mlp: fused kernel covers C=%d, hidden=%d (got %d, %d)", MC, MH, w->C,
                 w->hidden);
  SHRIMP_REQUIRE(w->out_w && w->out_b && w->g_attn && w->ln_w && w->ln_b && w->fc1_w &&
                     w->fc1_b && w->fc2_w && w->fc2_b && w->g_mlp,
                 "pack_attn_mlp: null weight pointer");
  hipStream_t st = as_stream(stream);
  unsigned char* pk = static_cast<unsigned char*>(packed);
  float* tmp = static_cast<float*>(scratch);  // MC * MH floats
  struct Part {
    const float* src; const float* rs; const float* cs; int n_out, n_in; uint32_t off; int il;
  } parts[3] = {{w->out_w, w->g_attn, nullptr, MC, MC, WO_OFF, 0},
                {w->fc1_w, nullptr, w->ln_w, MH, MC, W1_OFF, 1},
                {w->fc2_w, w->g_mlp, nullptr, MC, MH, W2_OFF, 1}};
  for (const Part& p : parts) {
    const int64_t n = (int64_t)p.n_out * p.n_in;
    hipLaunchKernelGGL(scale_rows_cols_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       p.src, p.rs, p.cs, p.n_out, p.n_in, tmp);
    const int64_t frags = (int64_t)(p.n_in / 32) * (p.n_out / 16) * 64;
    hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((frags + 255) / 256)), dim3(256), 0, st,
                       tmp, reinterpret_cast<unsigned short*>(pk + p.off), p.n_in, p.n_out, p.n_in,
                       p.n_in, (int64_t)0, (int64_t)1, (int64_t)p.n_in, p.il);
  }
  hipLaunchKernelGGL(attn_mlp_bias_kernel, dim3((MC + MH + MC + 255) / 256), dim3(256), 0, st, *w,
                     reinterpret_cast<float*>(pk + BO_OFF));
  return check_launch("pack_attn_mlp");
}

extern "C" int shrimp_attn_mlp(const shrimp_mlp_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_mlp: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "attn_mlp: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->C == MC && a->hidden == MH,
                 "attn_mlp: fused kernel covers C=%d, hidden=%d (got C=%d, hidden=%d)", MC, MH,
                 a->C, a->hidden);
  SHRIMP_REQUIRE(a->x && a->seq && a->mask && a->packed, "attn_mlp: null pointer");
  SHRIMP_REQUIRE(strides_ok({a->x_sr, a->s_sr}), "attn_mlp: row strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->x_sr >= MC && a->x_sr % 8 == 0 && a->s_sr >= MC && a->s_sr % 8 == 0,
                 "attn_mlp: row strides must be >= C and multiples of 8");
  const int64_t xe = ((int64_t)(a->rows - 1) * a->x_sr + MC) * 2;
  const int64_t se = ((int64_t)(a->rows - 1) * a->s_sr + MC) * 2;
  SHRIMP_REQUIRE(xe < (int64_t)0x7FFF0000 && se < (int64_t)0x7FFF0000,
                 "attn_mlp: activation buffer too large");
  SHRIMP_REQUIRE(a->S > 0 && a->rows % a->S == 0 && a->n_tokens >= 0 && a->n_tokens <= a->S,
                 "attn_mlp: rows must be whole positions of S rows (rows %d, S %d, tokens %d)",
                 a->rows, a->S, a->n_tokens);
  const int64_t lob = a->tok_lo ? (int64_t)(a->rows / a->S) * a->n_tokens * MC * 2 : 0;
  SHRIMP_REQUIRE(lob < (int64_t)0x7FFF0000, "attn_mlp: token low parts too large");
  SHRIMP_REQUIRE((size_t)max_lds_per_block() >= W_LDS,
                 "attn_mlp: needs %u bytes of LDS per workgroup", (unsigned)W_LDS);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return set_error(SHRIMP_ELAUNCH, "attn_mlp: cannot query the compute unit count");
  const int64_t nblk = (a->rows + 15) / 16;
  // at least one workgroup per 4 row blocks (up to one per compute unit): small
  // row counts spread over more units, each staging the weights once
  const int grid = (int)std::min<int64_t>(cus, std::max<int64_t>((nblk + MWAVES - 1) / MWAVES, (nblk + 3) / 4));
  hipLaunchKernelGGL(attn_mlp_kernel, dim3(grid), dim3(MWAVES * 64), W_LDS, as_stream(stream), *a,
                     (uint32_t)xe, (uint32_t)se, (uint32_t)lob);
  return check_launch("attn_mlp");
}
