// fp32 serve mode and the chunked attention fallback.
//
// The reference serves in fp32 when autocast is off (SHRIMP_SERVE_AUTOCAST=0,
// packages/shrimp/python/shrimp/inference.py:50-68). These kernels run the
// same forward as the bf16 kernels with fp32 activations end to end:
//
//  * gemm32x3_kernel / gemm32_kernel (one body, gemm32_body): the
//    gather-GEMM hex conv (HexNodeConv / hex_conv_ln, model.py:346-370,
//    395-422; _triton_conv.py:46-196) and the nn.Linear row GEMMs of the
//    attention block (model.py:448-514), with every epilogue of the bf16
//    kernels (bias, LayerNorm, ReLU, row mask, ConvBlock residual,
//    LayerScale residual, GELU, q/k/v head split, policy head) and a
//    LayerNorm prologue for the linear inputs. Input widths that are
//    multiples of 32 run gemm32x3_kernel: bf16 MFMA on hi / lo split
//    operands (see gemm32_body). The 16-channel stem runs gemm32_kernel on
//    v_mfma_f32_16x16x4_f32.
//    Orientation as in the bf16 kernels: out^T = W^T . X^T, so lane (lr, lg)
//    of a 16x16 result holds outputs 4 lg .. +3 of row lr. In the fp32
//    kernel a k-chunk is 16 input channels: lane group lg loads channels
//    4 lg .. +3 of its row as one 16-byte load, and MFMA step s (0..3) of
//    the chunk takes channel 4 lg + s as k slot lg. Weights are packed to
//    match (16-byte fragments).
//  * attn32_mfma_kernel: the fp32 attention at head dim 16 (coords mode) on
//    bf16 MFMA with hi / lo operand splitting (see the kernel);
//  * attn_rows_kernel: softmax(q k^T / sqrt(d) + bias) v with one query row
//    per thread and keys streamed through LDS in chunks, so any sequence
//    length fits (the fused bf16 kernel stages the whole sequence). fp32
//    scores, statistics and accumulators; q/k/v/out fp32 or bf16.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

#define SHRIMP_LOG2E_F32 1.4426950408889634f
#define SHRIMP_NEG_BIG_F32 (-1.0e30f)

SHRIMP_DEV f32x4 as_f32x4(u32x4 v) { return __builtin_bit_cast(f32x4, v); }

SHRIMP_DEV f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---- fp32 gather / row GEMM ------------------------------------------------------

enum : int {
  G_GATHER = 1,  // rows gathered through idx (conv); else row n of position b
  G_PLN = 2,     // LayerNorm prologue on the input rows (linear)
  G_LN = 4,      // LayerNorm over the outputs (conv)
  G_RELU = 8,
  G_MASK = 16,   // conv: rows with mask 0 give 0 (after LayerNorm / ReLU)
  G_CRES = 32,   // ConvBlock residual: out = relu(resid + gamma * y)
  G_LRES = 64,   // LayerScale residual: out = resid + gamma * (mask ? y : 0)
  G_GELU = 128,
  G_QKV = 256,   // q / k / v split into (3, B, H, S, dpad)
  G_HEAD = 512,  // policy head: head_out = mask ? relu(acc) . head_w + head_b : 0
};

struct Gemm32 {
  const float* x;
  int64_t x_sb, x_sr;  // elements between positions / rows
  uint32_t x_bytes;
  const int32_t* idx;  // gather: (B, N, idx_stride)
  int taps, idx_stride;
  const uint8_t* mask;  // (B * N) or NULL
  const float* w;       // packed
  const float* bias;
  const float* ln_w;
  const float* ln_b;
  float eps;
  const float* resid;
  int64_t r_sb, r_sr;
  const float* gamma;
  const float* head_w;
  const float* head_b;
  float* head_out;
  float* out;
  int64_t o_sb, o_sr;
  int B, N;   // rows are (b, n), b < B, n < N (linear: N = 1)
  int kin;    // input channels per tap (multiple of 16)
  int cout;   // multiple of 16
  int S, H, dpad;  // QKV split: row = b * N + n is sequence row (r / S, r % S)
};

// One wave: MB x 16 rows by NB x 16 outputs at a time (blockIdx.y selects the
// output blocks, or the workgroup walks them all: YLOOP); four waves per
// workgroup.
// X3 (kin a multiple of 32): the products on bf16 MFMA with each fp32 operand
// split as x = hi + lo (hi = bf16(x), lo = bf16(x - hi)), a 16 x 16 x 32 tile
// taken as hi·lo + lo·hi + hi·hi (the lo·lo term is below 2^-16 of the
// product): relative error near 2^-16 per product against fp32 products, at
// 16x the fp32 MFMA rate. The weights come packed as hi / lo fragments
// (pack_w32x3_kernel); x is split as it is loaded, lane group lg taking
// channels 8 lg .. + 7 of each 32-channel chunk.
template <int NB, int MB, int F, bool X3>
SHRIMP_DEV void gemm32_body(const Gemm32& g) {
  constexpr bool GATHER = (F & G_GATHER) != 0, PLN = (F & G_PLN) != 0;
  constexpr bool LN = (F & G_LN) != 0, RELU = (F & G_RELU) != 0, MASK = (F & G_MASK) != 0;
  constexpr bool CRES = (F & G_CRES) != 0, LRES = (F & G_LRES) != 0;
  constexpr bool GELU = (F & G_GELU) != 0, QKV = (F & G_QKV) != 0, HEAD = (F & G_HEAD) != 0;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int64_t R = (int64_t)g.B * g.N;
  const int64_t row_base = ((int64_t)blockIdx.x * 4 + wave) * (MB * 16);
  // X3 waves share weight fragments through LDS with a barrier per stage, so
  // a wave past the last row stays until the K loop ends.
  if (!X3 && row_base >= R) return;
  // With a LayerNorm prologue the split kernel walks all output blocks itself
  // (grid.y 1), so the rows come from HBM and their statistics are taken once.
  constexpr bool YLOOP = X3 && PLN;
  const int NBT = g.cout / 16;
  const int KC = g.kin / 16;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, g.x_bytes);

  int rb[MB], rn[MB];
  bool rv[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t r = row_base + mb * 16 + lr;
    rv[mb] = r < R;
    rb[mb] = rv[mb] ? (int)(r / g.N) : 0;
    rn[mb] = rv[mb] ? (int)(r - (int64_t)rb[mb] * g.N) : 0;
  }

  // LayerNorm statistics of the input rows (two passes over the row; each
  // pass requests four 16-channel chunks of every row block at a time, the
  // sums still taken chunk by chunk in order)
  float pmean[MB], prstd[MB];
  if constexpr (PLN) {
    uint32_t off[MB];
    float s[MB], q[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      off[mb] = rv[mb] ? (uint32_t)(((int64_t)rb[mb] * g.x_sb + (int64_t)rn[mb] * g.x_sr) * 4) +
                             (uint32_t)(lg * 16)
                       : SHRIMP_OOB_OFFSET;
      s[mb] = 0.f;
      q[mb] = 0.f;
    }
    auto pass = [&](auto&& use) {
      int kc = 0;
      for (; kc + 4 <= KC; kc += 4) {
        f32x4 v[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int u = 0; u < 4; ++u) v[mb][u] = as_f32x4(buf_load16(xr, off[mb] + (kc + u) * 64));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int u = 0; u < 4; ++u) use(mb, v[mb][u]);
      }
      for (; kc < KC; ++kc)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) use(mb, as_f32x4(buf_load16(xr, off[mb] + kc * 64)));
    };
    pass([&](int mb, const f32x4& v) { s[mb] += (v[0] + v[1]) + (v[2] + v[3]); });
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) pmean[mb] = sum_lane_groups(s[mb]) / (float)g.kin;
    pass([&](int mb, const f32x4& v) {
#pragma unroll
      for (int j = 0; j < 4; ++j) q[mb] = fmaf(v[j] - pmean[mb], v[j] - pmean[mb], q[mb]);
    });
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) prstd[mb] = rsqrtf(sum_lane_groups(q[mb]) / (float)g.kin + g.eps);
  }

  for (int yb = 0; yb < (YLOOP ? NBT / NB : 1); ++yb) {
  const int nb0 = (YLOOP ? yb : (int)blockIdx.y) * NB;
  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int T = GATHER ? g.taps : 1;
  // X3: a chunk's NB hi / lo fragment pairs (NB x 2 KiB, contiguous in the
  // packed weights) are loaded once per workgroup, 16 bytes per thread at a
  // time, into one of two LDS buffers; the waves read their lane's fragments
  // from there. A buffer (stage) holds SD consecutive chunks, so the waves
  // meet at a barrier once per SD chunks.
  constexpr int SD = NB <= 8 ? 2 : 1;  // chunks per stage (64 KiB of LDS at NB = 8)
  constexpr int CW = NB * 128;         // 16-byte pieces per chunk
  constexpr int SPT = X3 ? (SD * CW + 255) / 256 : 1;  // staging loads per thread
  __shared__ u32x4 wsh[X3 ? 2 : 1][X3 ? SD * CW : 1];
  u32x4 stg[SPT];
  const int NC = X3 ? T * (g.kin / 32) : 0;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(g.w, X3 ? (uint32_t)((int64_t)NC * NBT * 2048) : 0u);
  auto stage_load = [&](int st) {  // chunks SD st .. + SD - 1, past the last one reloading it
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int i = threadIdx.x + k * 256;
      if ((SD * CW) % 256 == 0 || i < SD * CW) {
        const int cc = min(st * SD + i / CW, NC - 1);
        stg[k] = buf_load16(wr, (uint32_t)(cc * NBT + nb0) * 2048u + (uint32_t)(i % CW) * 16u);
      }
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int i = threadIdx.x + k * 256;
      if ((SD * CW) % 256 == 0 || i < SD * CW) wsh[buf][i] = stg[k];
    }
  };
  if constexpr (X3) {
    // Flat K loop over 32-channel chunks (tap t, chunk kc of KC2). Chunk c
    // requests chunk c + 1's x rows; the first chunk of a stage also requests
    // the next stage's weight fragments into the staging registers, which
    // the stage's last chunk stores to the other LDS buffer before the
    // barrier. So every chunk starts with its rows and fragments in place. A
    // tap's gather indices are requested during the first chunk of the tap
    // before (past the last chunk, loads reload the last one).
    const int KC2 = g.kin / 32;
    int jn[MB];
    uint32_t xo[MB];
    auto tap_idx = [&](int t) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        jn[mb] = rn[mb];
        if (GATHER) jn[mb] = rv[mb] ? g.idx[((int64_t)rb[mb] * g.N + rn[mb]) * g.idx_stride + t] : -1;
        SHRIMP_DCHECK(!GATHER || jn[mb] >= -1, SHRIMP_DBG_CONV_INDEX);
      }
    };
    auto tap_off = [&]() {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bool ok = rv[mb] && jn[mb] >= 0 && jn[mb] < g.N;
        xo[mb] = ok ? (uint32_t)(((int64_t)rb[mb] * g.x_sb + (int64_t)jn[mb] * g.x_sr) * 4) +
                          (uint32_t)(lg * 32)
                    : SHRIMP_OOB_OFFSET;
      }
    };
    auto xload = [&](int kc, f32x4(&x)[MB][2]) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        x[mb][0] = as_f32x4(buf_load16(xr, xo[mb] + kc * 128));
        x[mb][1] = as_f32x4(buf_load16(xr, xo[mb] + kc * 128 + 16));
      }
    };
    int t = 0, kc = 0;  // the chunk being computed
    // even: c is the first chunk of its pair (a compile-time constant per call)
    auto step = [&](int c, bool even, const f32x4(&xv)[MB][2], f32x4(&xn)[MB][2]) {
      const int kcc = kc, tc = t;
      // The next tap's indices go out after this step's rows and fragments
      // (so waiting for those never waits for them), except with one chunk
      // per tap, where the next step already needs them.
      if (KC2 == 1 && tc + 1 < T) tap_idx(tc + 1);
      if (++kc == KC2) {
        kc = 0;
        if (++t < T) tap_off();
        else { t = T - 1; kc = KC2 - 1; }  // past the end: reload the last chunk
      }
      xload(kc, xn);
      if (SD == 1 || even) stage_load(c / SD + 1);
      if (KC2 > 1 && kcc == 0 && tc + 1 < T) tap_idx(tc + 1);
      __builtin_amdgcn_sched_barrier(0);
      u32x4 wh[NB], wl[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        wh[nb] = wsh[(c / SD) & 1][(c % SD) * CW + (nb * 2) * 64 + lane];
        wl[nb] = wsh[(c / SD) & 1][(c % SD) * CW + (nb * 2 + 1) * 64 + lane];
      }
      u32x4 xh[MB], xl[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float x[8] = {xv[mb][0][0], xv[mb][0][1], xv[mb][0][2], xv[mb][0][3],
                      xv[mb][1][0], xv[mb][1][1], xv[mb][1][2], xv[mb][1][3]};
        if constexpr (PLN) {
          const int ch = kcc * 32 + lg * 8;
          const f32x4 lw0 = *reinterpret_cast<const f32x4*>(g.ln_w + ch);
          const f32x4 lw1 = *reinterpret_cast<const f32x4*>(g.ln_w + ch + 4);
          const f32x4 lb0 = *reinterpret_cast<const f32x4*>(g.ln_b + ch);
          const f32x4 lb1 = *reinterpret_cast<const f32x4*>(g.ln_b + ch + 4);
          const float lw[8] = {lw0[0], lw0[1], lw0[2], lw0[3], lw1[0], lw1[1], lw1[2], lw1[3]};
          const float lb[8] = {lb0[0], lb0[1], lb0[2], lb0[3], lb1[0], lb1[1], lb1[2], lb1[3]};
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = fmaf((x[e] - pmean[mb]) * prstd[mb], lw[e], lb[e]);
        }
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          const unsigned hw = pack_bf16x2(x[2 * w2], x[2 * w2 + 1]);
          xh[mb][w2] = hw;
          xl[mb][w2] = pack_bf16x2(x[2 * w2] - bf16_lo(hw), x[2 * w2 + 1] - bf16_hi(hw));
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          acc[nb][mb] = mfma16x16x32(wh[nb], xl[mb], acc[nb][mb]);
          acc[nb][mb] = mfma16x16x32(wl[nb], xh[mb], acc[nb][mb]);
          acc[nb][mb] = mfma16x16x32(wh[nb], xh[mb], acc[nb][mb]);
        }
      }
      // The other buffer was last read in the previous stage, before the
      // previous barrier; the barrier below publishes it for the next stage.
      if (SD == 1 || !even) {
        stage_store((c / SD + 1) & 1);
        __syncthreads();
      }
    };
    f32x4 xa[MB][2], xb[MB][2];
    tap_idx(0);
    tap_off();
    xload(0, xa);
    stage_load(0);
    stage_store(0);
    __syncthreads();
    int c = 0;
    for (; c + 1 < NC; c += 2) {
      step(c, true, xa, xb);
      step(c + 1, false, xb, xa);
    }
    if (c < NC) step(c, true, xa, xb);
  }
  if constexpr (!X3) {
  // fp32 fragments on v_mfma_f32_16x16x4f32, 16 input channels per k-chunk
  const f32x4* wp = reinterpret_cast<const f32x4*>(g.w);
  for (int t = 0; t < T; ++t) {
    uint32_t xoff[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      int j = rn[mb];
      if (GATHER) j = rv[mb] ? g.idx[((int64_t)rb[mb] * g.N + rn[mb]) * g.idx_stride + t] : -1;
      SHRIMP_DCHECK(!GATHER || j >= -1, SHRIMP_DBG_CONV_INDEX);
      const bool ok = rv[mb] && j >= 0 && j < g.N;
      xoff[mb] = ok ? (uint32_t)(((int64_t)rb[mb] * g.x_sb + (int64_t)j * g.x_sr) * 4) +
                          (uint32_t)(lg * 16)
                    : SHRIMP_OOB_OFFSET;
    }
    for (int kc = 0; kc < KC; ++kc) {
      f32x4 bx[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) bx[mb] = as_f32x4(buf_load16(xr, xoff[mb] + kc * 64));
      if constexpr (PLN) {
        const int c = kc * 16 + lg * 4;
        const f32x4 lw = *reinterpret_cast<const f32x4*>(g.ln_w + c);
        const f32x4 lb = *reinterpret_cast<const f32x4*>(g.ln_b + c);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j) bx[mb][j] = fmaf((bx[mb][j] - pmean[mb]) * prstd[mb], lw[j], lb[j]);
      }
      f32x4 aw[NB];
      const int64_t kb = ((int64_t)t * KC + kc) * NBT;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) aw[nb] = wp[(kb + nb0 + nb) * 64 + lane];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma16x16x4f32(aw[nb][s], bx[mb][s], acc[nb][mb]);
    }
  }
  }  // !X3

  if (row_base >= R) {
    if constexpr (YLOOP) continue;  // the next output block's barriers need the wave
    else return;
  }
  // ---- epilogue: lane (lr, lg) holds outputs 16 (nb0 + nb) + 4 lg + j of row lr --------
  const float inv_cout = 1.0f / (float)g.cout;
  const float hb = HEAD ? g.head_b[0] : 0.f;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t rowi = (int64_t)rb[mb] * g.N + rn[mb];
    const bool live = rv[mb] && (g.mask == nullptr || g.mask[rowi] != 0);
    float y[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 bb = *reinterpret_cast<const f32x4*>(g.bias + (nb0 + nb) * 16 + lg * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) y[nb][j] = acc[nb][mb][j] + bb[j];
    }
    if constexpr (HEAD) {
      float s = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 hw = *reinterpret_cast<const f32x4*>(g.head_w + nb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) s = fmaf(fmaxf(y[nb][j], 0.f), hw[j], s);
      }
      s = sum_lane_groups(s);
      if (rv[mb] && lg == 0) g.head_out[rowi] = live ? s + hb : 0.f;
      continue;
    }
    if constexpr (LN) {
      float s = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += y[nb][j];
      const float mean = sum_lane_groups(s) * inv_cout;
      float q = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) q = fmaf(y[nb][j] - mean, y[nb][j] - mean, q);
      const float rstd = rsqrtf(sum_lane_groups(q) * inv_cout + g.eps);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 lw = *reinterpret_cast<const f32x4*>(g.ln_w + nb * 16 + lg * 4);
        const f32x4 lb = *reinterpret_cast<const f32x4*>(g.ln_b + nb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) y[nb][j] = fmaf((y[nb][j] - mean) * rstd, lw[j], lb[j]);
      }
    }
    if (!rv[mb]) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = (nb0 + nb) * 16 + lg * 4;
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = y[nb][j];
        if (GELU) v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
        if (RELU) v = fmaxf(v, 0.f);
        if (MASK) v = live ? v : 0.f;
        o[j] = v;
      }
      if constexpr (CRES || LRES) {
        const f32x4 rr = *reinterpret_cast<const f32x4*>(g.resid + (int64_t)rb[mb] * g.r_sb +
                                                           (int64_t)rn[mb] * g.r_sr + n);
        const f32x4 gm = *reinterpret_cast<const f32x4*>(g.gamma + n);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (CRES) o[j] = fmaxf(rr[j] + gm[j] * o[j], 0.f);
          else o[j] = rr[j] + gm[j] * (live ? o[j] : 0.f);
        }
      }
      float* dst;
      if constexpr (QKV) {
        const int C3 = g.cout / 3;
        const int which = n / C3;
        const int nn = n - which * C3;
        const int dh = C3 / g.H;
        const int hh = nn / dh;
        const int dd = nn - hh * dh;
        const int bq = (int)(rowi / g.S);
        const int sq = (int)(rowi - (int64_t)bq * g.S);
        const int64_t nbq = R / g.S;
        dst = g.out + ((((int64_t)which * nbq + bq) * g.H + hh) * g.S + sq) * g.dpad + dd;
      } else {
        dst = g.out + (int64_t)rb[mb] * g.o_sb + (int64_t)rn[mb] * g.o_sr + n;
      }
      *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
    }
  }
  }  // output blocks
}

// The split-operand kernels keep two waves per SIMD (at most 256 registers);
// the fp32-fragment kernel (16-channel inputs) keeps the default bound.
template <int NB, int MB, int F>
__global__ __launch_bounds__(256, 2) void gemm32x3_kernel(const Gemm32 g) {
  gemm32_body<NB, MB, F, true>(g);
}
template <int NB, int MB, int F>
__global__ __launch_bounds__(256) void gemm32_kernel(const Gemm32 g) {
  gemm32_body<NB, MB, F, false>(g);
}

// Packs W (K x cout, element (k, n) at w[k * sk + n * sn], k = t * kin + c
// for c < kin_real and zero for kin_real <= c < kin) into 16-byte fragments:
// fragment (kc, nb) lane (lr, lg) = W[16 kc + 4 lg + j][16 nb + lr], j < 4.
__global__ void pack_w32_kernel(const float* __restrict__ w, float* __restrict__ packed, int taps,
                                int kin_real, int kin, int cout, int64_t st, int64_t sk,
                                int64_t sn) {
  const int64_t total = (int64_t)taps * kin * cout;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int j = (int)(i & 3);
  const int lane = (int)((i >> 2) & 63);
  const int64_t frag = i >> 8;
  const int NBT = cout / 16;
  const int nb = (int)(frag % NBT);
  const int64_t kcg = frag / NBT;  // global k-chunk: t * (kin / 16) + kc
  const int kcpt = kin / 16;
  const int t = (int)(kcg / kcpt);
  const int c = (int)(kcg - (int64_t)t * kcpt) * 16 + (lane >> 4) * 4 + j;
  const int n = nb * 16 + (lane & 15);
  packed[i] = c < kin_real ? w[(int64_t)t * st + (int64_t)c * sk + (int64_t)n * sn] : 0.f;
}

// The same weights for the X3 path (kin a multiple of 32), in the bytes of the
// fp32 layout: per (32-row k-chunk kc, output block nb) a 1 KiB hi fragment
// and a 1 KiB lo fragment, lane (lr, lg) holding W[32 kc + 8 lg + e][16 nb +
// lr], e < 8, as bf16 (hi = bf16(w), lo = bf16(w - hi)).
__global__ void pack_w32x3_kernel(const float* __restrict__ w, unsigned short* __restrict__ packed,
                                  int taps, int kin_real, int kin, int cout, int64_t st, int64_t sk,
                                  int64_t sn) {
  const int64_t total = (int64_t)taps * kin * cout;  // weights; each one a hi and a lo element
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int e = (int)(i & 7);
  const int lane = (int)((i >> 3) & 63);
  const int64_t frag = i >> 9;  // (t, kc, nb)
  const int NBT = cout / 16;
  const int nb = (int)(frag % NBT);
  const int64_t kcg = frag / NBT;
  const int kcpt = kin / 32;
  const int t = (int)(kcg / kcpt);
  const int c = (int)(kcg - (int64_t)t * kcpt) * 32 + (lane >> 4) * 8 + e;
  const int n = nb * 16 + (lane & 15);
  const float v = c < kin_real ? w[(int64_t)t * st + (int64_t)c * sk + (int64_t)n * sn] : 0.f;
  const unsigned short hi = f32_to_bf16_bits(v);
  const unsigned short lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
  packed[frag * 1024 + lane * 8 + e] = hi;
  packed[frag * 1024 + 512 + lane * 8 + e] = lo;
}

template <int NB, int MB, int F>
static int launch_gemm32(const Gemm32& g, hipStream_t st) {
  const int64_t R = (int64_t)g.B * g.N;
  const int64_t per = 4 * MB * 16;
  const bool yloop = (F & G_PLN) != 0 && g.kin % 32 == 0;  // gemm32_body's YLOOP
  dim3 grid((unsigned)((R + per - 1) / per), yloop ? 1u : (unsigned)(g.cout / 16 / NB));
  if (g.kin % 32 == 0)
    hipLaunchKernelGGL((gemm32x3_kernel<NB, MB, F>), grid, dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((gemm32_kernel<NB, MB, F>), grid, dim3(256), 0, st, g);
  return check_launch("gemm32");
}

// Packs into the layout the kernel reads for this kin: hi / lo bf16
// fragments when kin is a multiple of 32, fp32 fragments otherwise.
static int pack_w32(const float* w, float* packed, int taps, int kin_real, int kin, int cout,
                    int64_t st, int64_t sk, int64_t sn, hipStream_t stream) {
  const int64_t total = (int64_t)taps * kin * cout;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (kin % 32 == 0)
    hipLaunchKernelGGL(pack_w32x3_kernel, grid, dim3(256), 0, stream, w,
                       reinterpret_cast<unsigned short*>(packed), taps, kin_real, kin, cout, st, sk,
                       sn);
  else
    hipLaunchKernelGGL(pack_w32_kernel, grid, dim3(256), 0, stream, w, packed, taps, kin_real,
                       kin, cout, st, sk, sn);
  return SHRIMP_OK;
}

// Every output block in one wave (LayerNorm, head epilogues): NB = cout / 16.
template <int F>
static int dispatch_full(const Gemm32& g, hipStream_t st) {
  switch (g.cout / 16) {
    case 2: return launch_gemm32<2, 4, F>(g, st);
    case 4: return launch_gemm32<4, 4, F>(g, st);
    case 6: return launch_gemm32<6, 2, F>(g, st);
    case 8: return launch_gemm32<8, 2, F>(g, st);
    case 12: return launch_gemm32<12, 1, F>(g, st);
    case 16: return launch_gemm32<16, 1, F>(g, st);
    default:
      return set_error(SHRIMP_EINVAL, "fp32 gemm: %d output channels with a LayerNorm / head "
                       "epilogue (supported: 32, 64, 96, 128, 192, 256)", g.cout);
  }
}

// Output blocks split over blockIdx.y.
template <int F>
static int dispatch_split(const Gemm32& g, hipStream_t st) {
  const int nbt = g.cout / 16;
  if (nbt % 8 == 0) return launch_gemm32<8, 2, F>(g, st);
  if (nbt % 6 == 0) return launch_gemm32<6, 2, F>(g, st);
  if (nbt % 4 == 0) return launch_gemm32<4, 4, F>(g, st);
  if (nbt % 2 == 0) return launch_gemm32<2, 4, F>(g, st);
  return launch_gemm32<1, 4, F>(g, st);
}

// ---- chunked attention --------------------------------------------------------------

template <typename T>
SHRIMP_DEV float load_act(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 4) return reinterpret_cast<const float*>(p)[i];
  else return bf16_bits_to_f32(reinterpret_cast<const unsigned short*>(p)[i]);
}
template <typename T>
SHRIMP_DEV void store_act(T* p, int64_t i, float v) {
  if constexpr (sizeof(T) == 4) reinterpret_cast<float*>(p)[i] = v;
  else reinterpret_cast<unsigned short*>(p)[i] = f32_to_bf16_bits(v);
}

constexpr int AR_THREADS = 128;  // query rows per workgroup
constexpr int AR_KC = 32;        // keys per staged chunk
// keys per online-softmax step (fewer at wide heads: registers)
constexpr int ar_kg(int dm) { return dm <= 16 ? 8 : (dm == 32 ? 4 : 2); }

// One thread per query row of one (position, head); keys in chunks of AR_KC
// staged in LDS (K, V rows, key class and coordinates). Bias sources as in
// shrimp_attn: pair rows of table2 (raw, log2e applied here) or the clamped
// offset LUT btab (log2e folded) with its three token rows.
template <typename T, int DM, bool PAIR>
__global__ __launch_bounds__(AR_THREADS) void attn_rows_kernel(const shrimp_attn_args a,
                                                              float qk_scale, int npos) {
  constexpr int AR_KG = ar_kg(DM);
  __shared__ __attribute__((aligned(16))) float ks[AR_KC][DM];
  __shared__ __attribute__((aligned(16))) float vs[AR_KC][DM];
  __shared__ int kq[AR_KC], kr[AR_KC], kcl[AR_KC];
  enum { K_CELL = 0, K_TOKEN = 1, K_DEAD = 2 };
  const int b = blockIdx.z;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int i = blockIdx.x * AR_THREADS + tid;
  const int S = a.S, d = a.d, nt = a.n_tokens, NC = S - nt;
  int L = a.seq_lens[b];
  SHRIMP_DCHECK(L >= 0 && L <= S, SHRIMP_DBG_SEQ_LEN);
  L = L < 0 ? 0 : (L > S ? S : L);
  const bool qv = i < L;
  const T* q = static_cast<const T*>(a.q) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  const T* k = static_cast<const T*>(a.k) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  const T* v = static_cast<const T*>(a.v) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  float qr[DM], acc[DM];
#pragma unroll
  for (int e = 0; e < DM; ++e) {
    qr[e] = (qv && e < d) ? load_act(q, (int64_t)i * a.dpad + e) * qk_scale : 0.f;
    acc[e] = 0.f;
  }
  const int M = a.lut_m, W = 2 * M + 1;
  const bool qtok = i < nt;
  int qq = 0, qrr = 0;
  if (!PAIR && qv && !qtok) {
    qq = a.coords[((int64_t)b * NC + (i - nt)) * 2];
    qrr = a.coords[((int64_t)b * NC + (i - nt)) * 2 + 1];
  }
  const uint8_t* prow = PAIR ? a.pair + (int64_t)b * a.p_sb + (int64_t)(qv ? i : 0) * a.p_sq : nullptr;
  float m = SHRIMP_NEG_BIG_F32, l = 0.f;
  for (int c0 = 0; c0 < L; c0 += AR_KC) {
    __syncthreads();
    for (int x = tid; x < AR_KC * DM; x += AR_THREADS) {
      const int kk = x / DM, e = x - kk * DM;
      const int key = c0 + kk;
      const bool ok = key < L && e < d;
      ks[kk][e] = ok ? load_act(k, (int64_t)key * a.dpad + e) : 0.f;
      vs[kk][e] = ok ? load_act(v, (int64_t)key * a.dpad + e) : 0.f;
    }
    if (tid < AR_KC) {
      const int key = c0 + tid;
      int cls = K_DEAD, cq = 0, cr = 0;
      if (key < L) {
        if (PAIR) {
          cls = K_CELL;
        } else if (key < nt) {
          cls = K_TOKEN;
        } else {
          const int64_t cell = (int64_t)b * NC + (key - nt);
          cls = a.mask[cell] ? K_CELL : K_DEAD;
          cq = a.coords[cell * 2];
          cr = a.coords[cell * 2 + 1];
        }
      }
      kcl[tid] = cls;
      kq[tid] = cq;
      kr[tid] = cr;
    }
    __syncthreads();
    if (!qv) continue;
    // groups of AR_KG keys: scores, then one online-softmax step
#pragma unroll 1
    for (int j0 = 0; j0 < AR_KC; j0 += AR_KG) {
      float sc[AR_KG];
      float cmax = SHRIMP_NEG_BIG_F32;
#pragma unroll
      for (int jj = 0; jj < AR_KG; ++jj) {
        const int j = j0 + jj;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < DM; ++e) s = fmaf(qr[e], ks[j][e], s);
        const int cls = kcl[j];
        float bias;
        if (PAIR) {
          int p = c0 + j < L ? (int)prow[c0 + j] : 0;
          p = p < npos ? p : npos - 1;
          bias = a.table2[(int64_t)p * a.H + h] * SHRIMP_LOG2E_F32;
        } else {
          int pos;
          if (cls == K_TOKEN) pos = qtok ? W * W + 2 : W * W;
          else if (qtok) pos = W * W + 1;
          else pos = (min(max(kq[j] - qq, -M), M) + M) * W + (min(max(kr[j] - qrr, -M), M) + M);
          bias = a.btab[(int64_t)pos * a.H + h];
        }
        s = cls == K_DEAD ? SHRIMP_NEG_BIG_F32 : s + bias;
        sc[jj] = s;
        cmax = fmaxf(cmax, s);
      }
      const float mnew = fmaxf(m, cmax);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int e = 0; e < DM; ++e) acc[e] *= alpha;
#pragma unroll
      for (int jj = 0; jj < AR_KG; ++jj) {
        const float p =
            sc[jj] > 0.5f * SHRIMP_NEG_BIG_F32 ? __builtin_amdgcn_exp2f(sc[jj] - mnew) : 0.f;
        l += p;
#pragma unroll
        for (int e = 0; e < DM; ++e) acc[e] = fmaf(p, vs[j0 + jj][e], acc[e]);
      }
    }
  }
  if (i >= S) return;
  T* o = static_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_sr;
  const float inv = (qv && l > 0.f) ? 1.0f / l : 0.f;
#pragma unroll
  for (int e = 0; e < DM; ++e)
    if (e < d) store_act(o, e, acc[e] * inv);
}

// fp32 attention at head dim 16 on bf16 MFMA, coords mode (the fp32 serve
// mode's attention; same semantics as attn_rows_kernel<float, 16, false>).
// Every fp32 operand x of a product is split as x = hi + lo with hi = bf16(x)
// and lo = bf16(x - hi), and a product of x and y takes the three MFMAs
// hi·hi + hi·lo + lo·hi (the lo·lo term is below 2^-16 of the product), with
// fp32 accumulation: relative error near 2^-16 against fp32 products, well
// inside the fp32 mode's 1e-4. One workgroup per (position, head), eight
// waves; K and V are staged once in LDS as hi / lo fragments in MFMA order
// (K fragment of key block kb: lane (lr, lg) holds K[16 kb + lr][4 lg .. + 3];
// V^T fragment: lane (lr, lg) holds V[16 kb + 4 lg .. + 3][lr]); each wave
// walks 16-query blocks over 16-key blocks with S^T = K Q^T (scale folded into
// q), an fp32 online softmax in base 2, and O^T += V^T P^T. The bias comes
// from an unclamped 53 x 53 copy of the head's LUT table when the position's
// cells inside the key bound (masked ones too: a masked query row still gets
// its attention, with its own coordinates) span at most 26 in q and r (one
// LDS read at key code - query code), else from the clamped table.
constexpr int A32_XD = 26, A32_XW = 2 * A32_XD + 1;
constexpr int A32_NW = 8;  // waves per workgroup

__host__ __device__ inline size_t attn32_mfma_lds(int S) {
  const size_t SP = (size_t)((S + 15) & ~15);
  return SP * (4 * 32 + 4 * 4) + (size_t)(A32_XW * A32_XW + 3) * 4 + 16 + (SP / 16) * 4;
}

__global__ __launch_bounds__(A32_NW * 64) void attn32_mfma_kernel(const shrimp_attn_args a, float qk_scale) {
  constexpr int NT = A32_NW * 64;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  enum { K_CELL = 0, K_TOKEN = 1, K_DEAD = 2 };
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const int S = a.S, H = a.H, nt = a.n_tokens, NC = S - nt;
  const int SP = (S + 15) & ~15, NKB = SP / 16;
  int L = a.seq_lens[b];
  SHRIMP_DCHECK(L >= 0 && L <= S, SHRIMP_DBG_SEQ_LEN);
  L = L < 0 ? 0 : (L > S ? S : L);
  const int M = a.lut_m, W = 2 * M + 1;

  u32x2* khi = reinterpret_cast<u32x2*>(smem);
  u32x2* klo = khi + NKB * 64;
  u32x2* vhi = klo + NKB * 64;
  u32x2* vlo = vhi + NKB * 64;
  int* kq = reinterpret_cast<int*>(vlo + NKB * 64);
  int* kr = kq + SP;
  int* kcls = kr + SP;
  int* kcode = kcls + SP;
  float* tab = reinterpret_cast<float*>(kcode + SP);  // [XW*XW or W*W] + 3 token biases
  int* red = reinterpret_cast<int*>(tab + A32_XW * A32_XW + 3);  // qmin, qmax, rmin, rmax
  int* bspec = red + 4;  // [NKB]: key block holds a token or a dead key

  if (tid < 4) red[tid] = (tid & 1) ? -(1 << 30) : (1 << 30);
  const float* q = static_cast<const float*>(a.q) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  const float* k = static_cast<const float*>(a.k) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  const float* v = static_cast<const float*>(a.v) + (int64_t)b * a.qkv_sb + (int64_t)h * a.qkv_sh;
  __syncthreads();

  // ---- keys: class, coordinates, span of the cells inside the bound ----------
  int qmn = 1 << 30, qmx = -(1 << 30), rmn = 1 << 30, rmx = -(1 << 30);
  for (int key = tid; key < SP; key += NT) {
    int cls = K_DEAD, cq = 0, cr = 0;
    if (key < L) {
      if (key < nt) {
        cls = K_TOKEN;
      } else {
        const int64_t cell = (int64_t)b * NC + (key - nt);
        cls = a.mask[cell] ? K_CELL : K_DEAD;
        cq = a.coords[cell * 2];
        cr = a.coords[cell * 2 + 1];
        qmn = min(qmn, cq);
        qmx = max(qmx, cq);
        rmn = min(rmn, cr);
        rmx = max(rmx, cr);
      }
    }
    kcls[key] = cls;
    kq[key] = cq;
    kr[key] = cr;
  }
  atomicMin(&red[0], qmn);
  atomicMax(&red[1], qmx);
  atomicMin(&red[2], rmn);
  atomicMax(&red[3], rmx);

  // ---- K and V as hi / lo bf16 fragments ---------------------------------------
  // item (key, g): dims 4 g .. + 3 of one key; keys >= L stage zeros
  for (int it = tid; it < SP * 4; it += NT) {
    const int key = it >> 2, g = it & 3;
    f32x4 kv = f32x4{0.f, 0.f, 0.f, 0.f}, vv = kv;
    if (key < L) {
      kv = *reinterpret_cast<const f32x4*>(k + (int64_t)key * a.dpad + 4 * g);
      vv = *reinterpret_cast<const f32x4*>(v + (int64_t)key * a.dpad + 4 * g);
    }
    const int kb = key >> 4, kl = key & 15;
    u32x2 hi, lo;
    hi.x = pack_bf16x2(kv[0], kv[1]);
    hi.y = pack_bf16x2(kv[2], kv[3]);
    lo.x = pack_bf16x2(kv[0] - bf16_lo(hi.x), kv[1] - bf16_hi(hi.x));
    lo.y = pack_bf16x2(kv[2] - bf16_lo(hi.y), kv[3] - bf16_hi(hi.y));
    khi[kb * 64 + g * 16 + kl] = hi;
    klo[kb * 64 + g * 16 + kl] = lo;
    // V^T: element (dim 4 g + c, key) -> lane (4 g + c, (key & 15) >> 2), slot key & 3
    unsigned short* vh16 = reinterpret_cast<unsigned short*>(vhi);
    unsigned short* vl16 = reinterpret_cast<unsigned short*>(vlo);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int slot = ((kb * 64 + (kl >> 2) * 16 + 4 * g + c) << 2) + (key & 3);
      const unsigned short hb = f32_to_bf16_bits(vv[c]);
      vh16[slot] = hb;
      vl16[slot] = f32_to_bf16_bits(vv[c] - bf16_bits_to_f32(hb));
    }
  }
  __syncthreads();

  // ---- the head's bias table --------------------------------------------------
  const int q0 = red[0], r0 = red[2];
  const bool linear = red[0] <= red[1] && red[1] - red[0] <= A32_XD && red[3] - red[2] <= A32_XD;
  const int W2 = W * W;
  if (linear) {
    // T[dq + XD][dr + XD] = btab at the clamped offset (the same value)
    for (int i = tid; i < A32_XW * A32_XW; i += NT) {
      const int dq = i / A32_XW - A32_XD, dr = i % A32_XW - A32_XD;
      const int pos = (min(max(dq, -M), M) + M) * W + (min(max(dr, -M), M) + M);
      tab[i] = a.btab[(int64_t)pos * H + h];
    }
  } else {
    for (int i = tid; i < W2; i += NT) tab[i] = a.btab[(int64_t)i * H + h];
  }
  if (tid < 3) tab[A32_XW * A32_XW + tid] = a.btab[(int64_t)(W2 + tid) * H + h];
  // cells (masked ones too) at their own offsets; tokens and keys past the
  // bound at (q0, r0), a valid index (their biases are selected per key)
  for (int key = tid; key < SP; key += NT) {
    const bool cell = key >= nt && key < L;
    kcode[key] = ((cell ? kq[key] : q0) - q0) * A32_XW + ((cell ? kr[key] : r0) - r0);
  }
  for (int kb = tid; kb < NKB; kb += NT) {
    int sp = 0;
    for (int j = 0; j < 16; ++j) sp |= kcls[kb * 16 + j] != K_CELL;
    bspec[kb] = sp;
  }
  __syncthreads();
  const float t_ct = tab[A32_XW * A32_XW], t_tc = tab[A32_XW * A32_XW + 1],
              t_tt = tab[A32_XW * A32_XW + 2];

  // ---- query blocks -------------------------------------------------------------
  const int nqb = (L + 15) / 16, nkb = (L + 15) / 16;
  for (int qb = wave; qb < nqb; qb += A32_NW) {
    const int query = qb * 16 + lr;
    const bool qv = query < L, qtok = query < nt;
    const bool qtokb = qb * 16 < nt;  // the block holds token queries (wave-uniform)
    const bool qcell = qv && !qtok;
    const int qq = qcell ? kq[query] : q0, qr = qcell ? kr[query] : r0;
    // table index of key j = kcode[j] - qoff
    const int qoff = (qq - q0) * A32_XW + (qr - r0) - (A32_XD * A32_XW + A32_XD);
    f32x4 qs = f32x4{0.f, 0.f, 0.f, 0.f};
    if (qv) qs = *reinterpret_cast<const f32x4*>(q + (int64_t)query * a.dpad + 4 * lg);
    qs = qs * qk_scale;
    u32x2 qh, ql;
    qh.x = pack_bf16x2(qs[0], qs[1]);
    qh.y = pack_bf16x2(qs[2], qs[3]);
    ql.x = pack_bf16x2(qs[0] - bf16_lo(qh.x), qs[1] - bf16_hi(qh.x));
    ql.y = pack_bf16x2(qs[2] - bf16_lo(qh.y), qs[3] - bf16_hi(qh.y));
    // m: the row's offset; lp: this lane's share of the row sum (its four
    // keys of every block), summed over the lane groups once at the end
    float m = SHRIMP_NEG_BIG_F32, lp = 0.f;
    bool mset = false;  // every query of the block has its offset (wave-uniform)
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nkb; ++kb) {
      const int fs = kb * 64 + lg * 16 + lr;
      // keys 16 kb + 4 lg + j of query lr
      const int key0 = kb * 16 + lg * 4;
      float s[4];
      float mx = SHRIMP_NEG_BIG_F32;
      const bool plain = linear && !qtokb && !bspec[kb];
      if (plain) {
        // cell queries, cell keys only (wave-uniform): the accumulators
        // start at the keys' biases, one table read per key
        const int4 kc = *reinterpret_cast<const int4*>(kcode + key0);
        f32x4 sc = f32x4{tab[kc.x - qoff], tab[kc.y - qoff], tab[kc.z - qoff], tab[kc.w - qoff]};
        sc = mfma16x16x16(khi[fs], ql, sc);
        sc = mfma16x16x16(klo[fs], qh, sc);
        sc = mfma16x16x16(khi[fs], qh, sc);
        // Once every query of the block has an offset m, the tile keeps it:
        // p = exp2(s - m) needs no maximum, no rescale and no lane exchange
        // (any fixed offset gives the same softmax; the sums only have to
        // stay finite and in range, else the tile takes the maximum path).
        if (mset) {
          float p[4], ps = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[j] = __builtin_amdgcn_exp2f(sc[j] - m);
            ps += p[j];
          }
          if (__builtin_amdgcn_ballot_w64(!(ps < 0x1p62f)) == 0) {
            lp += ps;
            u32x2 ph, pl;
            ph.x = pack_bf16x2(p[0], p[1]);
            ph.y = pack_bf16x2(p[2], p[3]);
            pl.x = pack_bf16x2(p[0] - bf16_lo(ph.x), p[1] - bf16_hi(ph.x));
            pl.y = pack_bf16x2(p[2] - bf16_lo(ph.y), p[3] - bf16_hi(ph.y));
            o = mfma16x16x16(vhi[fs], pl, o);
            o = mfma16x16x16(vlo[fs], ph, o);
            o = mfma16x16x16(vhi[fs], ph, o);
            continue;
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s[j] = sc[j];
          mx = fmaxf(mx, s[j]);
        }
      } else {
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
        sc = mfma16x16x16(khi[fs], ql, sc);
        sc = mfma16x16x16(klo[fs], qh, sc);
        sc = mfma16x16x16(khi[fs], qh, sc);
        const int4 cl = *reinterpret_cast<const int4*>(kcls + key0);
        const int clv[4] = {cl.x, cl.y, cl.z, cl.w};
        // every key's table entry is read (in the linear table any key's
        // code gives an index inside it), then replaced for tokens and dead
        // keys by selects, so the tile runs without branches
        float tb[4];
        if (linear) {
          const int4 kc = *reinterpret_cast<const int4*>(kcode + key0);
          tb[0] = tab[kc.x - qoff];
          tb[1] = tab[kc.y - qoff];
          tb[2] = tab[kc.z - qoff];
          tb[3] = tab[kc.w - qoff];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = key0 + j;
            tb[j] = tab[(min(max(kq[key] - qq, -M), M) + M) * W + (min(max(kr[key] - qr, -M), M) + M)];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float bias = tb[j];
          bias = qtok ? t_tc : bias;
          bias = clv[j] == K_TOKEN ? (qtok ? t_tt : t_ct) : bias;
          s[j] = clv[j] == K_DEAD ? SHRIMP_NEG_BIG_F32 : sc[j] + bias;
          mx = fmaxf(mx, s[j]);
        }
      }
      mx = max_groups_swap(mx);
      const float mnew = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      mset = __builtin_amdgcn_ballot_w64(!(m > 0.5f * SHRIMP_NEG_BIG_F32)) == 0;
      float p[4], ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[j] = s[j] > 0.5f * SHRIMP_NEG_BIG_F32 ? __builtin_amdgcn_exp2f(s[j] - mnew) : 0.f;
        ps += p[j];
      }
      lp = lp * alpha + ps;
      u32x2 ph, pl;
      ph.x = pack_bf16x2(p[0], p[1]);
      ph.y = pack_bf16x2(p[2], p[3]);
      pl.x = pack_bf16x2(p[0] - bf16_lo(ph.x), p[1] - bf16_hi(ph.x));
      pl.y = pack_bf16x2(p[2] - bf16_lo(ph.y), p[3] - bf16_hi(ph.y));
      o = o * alpha;
      o = mfma16x16x16(vhi[fs], pl, o);
      o = mfma16x16x16(vlo[fs], ph, o);
      o = mfma16x16x16(vhi[fs], ph, o);
    }
    const float l = sum_groups_swap(lp);
    // lane (lr, lg): dims 4 lg .. + 3 of query lr
    if (query < S) {
      const float inv = (qv && l > 0.f) ? 1.0f / l : 0.f;
      float* op = static_cast<float*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
                  (int64_t)query * a.o_sr + 4 * lg;
      *reinterpret_cast<f32x4*>(op) = o * inv;
    }
  }
  // query rows past the live bound (whole blocks) store zeros
  for (int i = nqb * 16 * 4 + tid; i < S * 4; i += NT) {
    const int row = i >> 2, g = i & 3;
    float* op = static_cast<float*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
                (int64_t)row * a.o_sr + 4 * g;
    *reinterpret_cast<f32x4*>(op) = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

template <typename T, bool PAIR>
static int launch_attn_rows(const shrimp_attn_args* a, int npos, hipStream_t st) {
  const float qk_scale = SHRIMP_LOG2E_F32 / sqrtf((float)a->d);
  dim3 grid((a->S + AR_THREADS - 1) / AR_THREADS, a->H, a->B);
#define SHRIMP_AR(DMV)                                                                        \
  if (a->d <= DMV) {                                                                          \
    hipLaunchKernelGGL((attn_rows_kernel<T, DMV, PAIR>), grid, dim3(AR_THREADS), 0, st, *a, \
                       qk_scale, npos);                                                       \
    return check_launch("attn_rows");                                                         \
  }
  SHRIMP_AR(8)
  SHRIMP_AR(16)
  SHRIMP_AR(32)
  SHRIMP_AR(64)
#undef SHRIMP_AR
  return set_error(SHRIMP_EINVAL, "attn: head dim %d above 64", a->d);
}

// Shared argument checks of the chunked attention; elem = element bytes.
static int check_attn_rows(const shrimp_attn_args* a, int elem, int* npos) {
  SHRIMP_REQUIRE(a->q && a->k && a->v && a->o && a->seq_lens, "attn: null pointer");
  SHRIMP_REQUIRE(a->d > 0 && a->d <= 64 && a->d <= a->dpad, "attn: head dim %d / pad %d", a->d,
                 a->dpad);
  SHRIMP_REQUIRE(a->n_tokens >= 0 && a->n_tokens <= a->S, "attn: bad n_tokens");
  (void)elem;
  if (a->pair != nullptr) {
    SHRIMP_REQUIRE(a->table2 && a->table_rows > 0, "attn: pair mode needs table2");
    *npos = a->table_rows;
  } else {
    SHRIMP_REQUIRE(a->btab && a->lut_m >= 0 && a->lut_m <= 64, "attn: coords mode needs btab");
    SHRIMP_REQUIRE(a->n_tokens == a->S || (a->coords && a->mask),
                   "attn: coords mode needs coords and mask");
    *npos = 0;
  }
  return SHRIMP_OK;
}

int attn_rows_bf16(const shrimp_attn_args* a, hipStream_t st) {
  int npos = 0;
  if (int rc = check_attn_rows(a, 2, &npos)) return rc;
  return a->pair ? launch_attn_rows<uint16_t, true>(a, npos, st)
                 : launch_attn_rows<uint16_t, false>(a, npos, st);
}

// ---- small fp32-mode kernels -----------------------------------------------------------

// xin (B, N, 16) fp32: features zero-padded to 16 channels.
template <int DT>
SHRIMP_DEV float load_feat32(const void* p, int64_t i) {
  if constexpr (DT == SHRIMP_DT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == SHRIMP_DT_F16) return (float)static_cast<const _Float16*>(p)[i];
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__global__ void feats32_kernel(const void* __restrict__ feats, int nfeat, int64_t total,
                               float* __restrict__ xin) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int f = (int)(i & 15);
  const int64_t r = i >> 4;
  xin[i] = f < nfeat ? load_feat32<DT>(feats, r * nfeat + f) : 0.f;
}

__global__ void csr_feats32_kernel(const uint16_t* __restrict__ feats, int nfeat,
                                   const int64_t* __restrict__ offsets, int row0, int N,
                                   float* __restrict__ xin) {
  const int b = blockIdx.y;
  const int64_t o = offsets[row0 + b];
  const int64_t cnt = offsets[row0 + b + 1] - o;
  const int n = cnt < 0 ? 0 : (cnt > N ? N : (int)cnt);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < N * 16; i += gridDim.x * blockDim.x) {
    const int r = i >> 4, f = i & 15;
    xin[(int64_t)b * N * 16 + i] =
        (r < n && f < nfeat) ? (float)__builtin_bit_cast(_Float16, feats[(o + r) * nfeat + f]) : 0.f;
  }
}

__global__ void fill_tokens32_kernel(const float* __restrict__ tokens, int n, float* __restrict__ seq,
                                     int64_t seq_sb) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < n; i += blockDim.x) seq[(int64_t)b * seq_sb + i] = tokens[i];
}

}  // namespace shrimp

using namespace shrimp;

// ---- C ABI ------------------------------------------------------------------------------

// 0 for a shape whose packed weights would not fit a 32-bit buffer offset
extern "C" size_t shrimp_conv_wpack_bytes_f32(int taps, int cin_pad, int cout) {
  const int64_t n = mul_sat({taps, cin_pad, cout, 4});
  return taps > 0 && cin_pad > 0 && cout > 0 && n < (int64_t)0x7FFF0000 ? (size_t)n : 0;
}

extern "C" int shrimp_pack_conv_weight_f32(const float* w, float* packed, int taps, int cin,
                                           int cin_pad, int cout, void* stream) {
  SHRIMP_REQUIRE(w && packed, "pack_conv_weight_f32: null pointer");
  SHRIMP_REQUIRE(taps > 0 && cin > 0 && cin <= cin_pad && cin_pad % 16 == 0,
                 "pack_conv_weight_f32: bad taps/cin (%d, %d, %d)", taps, cin, cin_pad);
  SHRIMP_REQUIRE(cout > 0 && cout % 16 == 0 && shrimp_conv_wpack_bytes_f32(taps, cin_pad, cout) > 0,
                 "pack_conv_weight_f32: cout %d", cout);
  pack_w32(w, packed, taps, cin, cin_pad, cout, (int64_t)cin * cout, (int64_t)cout, (int64_t)1,
           as_stream(stream));
  return check_launch("pack_conv_weight_f32");
}

extern "C" int shrimp_pack_linear_weight_f32(const float* w, float* packed, int in_features,
                                             int out_features, void* stream) {
  SHRIMP_REQUIRE(w && packed, "pack_linear_weight_f32: null pointer");
  SHRIMP_REQUIRE(in_features > 0 && in_features % 16 == 0 && out_features > 0 &&
                     out_features % 16 == 0 && shrimp_conv_wpack_bytes_f32(1, in_features, out_features) > 0,
                 "pack_linear_weight_f32: shape (%d -> %d) needs multiples of 16", in_features,
                 out_features);
  pack_w32(w, packed, 1, in_features, in_features, out_features, (int64_t)0, (int64_t)1,
           (int64_t)in_features, as_stream(stream));
  return check_launch("pack_linear_weight_f32");
}

extern "C" int shrimp_hex_conv_f32(const shrimp_conv_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "hex_conv_f32: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->N > 0 && a->N <= kMaxDim, "hex_conv_f32: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->idx && a->mask && a->w && a->bias, "hex_conv_f32: null pointer");
  SHRIMP_REQUIRE(a->taps > 0 && a->taps <= a->idx_stride, "hex_conv_f32: taps / idx stride");
  SHRIMP_REQUIRE(a->cin_pad > 0 && a->cin_pad % 16 == 0 && a->cout > 0 && a->cout % 16 == 0,
                 "hex_conv_f32: cin_pad %d / cout %d must be multiples of 16", a->cin_pad, a->cout);
  SHRIMP_REQUIRE(strides_ok({a->x_sb, a->x_sn, a->o_sb, a->o_sn, a->r_sb, a->r_sn}),
                 "hex_conv_f32: strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->x_sn >= a->cin_pad && a->x_sn % 4 == 0 && a->x_sb % 4 == 0,
                 "hex_conv_f32: x strides");
  const bool ln = a->ln_w != nullptr, resid = a->resid != nullptr, head = a->head_w != nullptr;
  SHRIMP_REQUIRE(!ln || a->ln_b, "hex_conv_f32: ln_w without ln_b");
  const int64_t xe = (int64_t)(a->B - 1) * a->x_sb + (int64_t)(a->N - 1) * a->x_sn + a->cin_pad;
  SHRIMP_REQUIRE(xe * 4 < (int64_t)0x7FFF0000, "hex_conv_f32: activation buffer too large");
  Gemm32 g{};
  g.x = static_cast<const float*>(a->x);
  g.x_sb = a->x_sb;
  g.x_sr = a->x_sn;
  g.x_bytes = (uint32_t)(xe * 4);
  g.idx = a->idx;
  g.taps = a->taps;
  g.idx_stride = a->idx_stride;
  g.mask = a->mask;
  g.w = static_cast<const float*>(a->w);
  g.bias = a->bias;
  g.ln_w = a->ln_w;
  g.ln_b = a->ln_b;
  g.eps = a->eps;
  g.resid = static_cast<const float*>(a->resid);
  g.r_sb = a->r_sb;
  g.r_sr = a->r_sn;
  g.gamma = a->gamma;
  g.head_w = a->head_w;
  g.head_b = a->head_b;
  g.head_out = a->head_out;
  g.out = static_cast<float*>(a->out);
  g.o_sb = a->o_sb;
  g.o_sr = a->o_sn;
  g.B = a->B;
  g.N = a->N;
  g.kin = a->cin_pad;
  g.cout = a->cout;
  hipStream_t st = as_stream(stream);
  if (head) {
    SHRIMP_REQUIRE(a->relu && a->head_b && a->head_out, "hex_conv_f32: head epilogue expects relu");
    return dispatch_full<G_GATHER | G_RELU | G_HEAD>(g, st);
  }
  SHRIMP_REQUIRE(a->out && a->o_sn % 4 == 0 && a->o_sb % 4 == 0, "hex_conv_f32: out strides");
  if (resid) {
    SHRIMP_REQUIRE(ln && !a->relu && a->gamma && a->r_sn % 4 == 0 && a->r_sb % 4 == 0,
                   "hex_conv_f32: residual epilogue is LN (no relu) + residual");
    return dispatch_full<G_GATHER | G_LN | G_MASK | G_CRES>(g, st);
  }
  if (ln)
    return a->relu ? dispatch_full<G_GATHER | G_LN | G_RELU | G_MASK>(g, st)
                   : dispatch_full<G_GATHER | G_LN | G_MASK>(g, st);
  return a->relu ? dispatch_split<G_GATHER | G_RELU | G_MASK>(g, st)
                 : dispatch_split<G_GATHER | G_MASK>(g, st);
}

extern "C" int shrimp_linear_f32(const shrimp_linear_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "linear_f32: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "linear_f32: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->w && a->bias && a->out, "linear_f32: null pointer");
  SHRIMP_REQUIRE(a->in_features % 16 == 0 && a->out_features % 16 == 0,
                 "linear_f32: in %d / out %d must be multiples of 16", a->in_features,
                 a->out_features);
  SHRIMP_REQUIRE(strides_ok({a->x_sr, a->o_sr, a->r_sr}), "linear_f32: row strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->x_sr >= a->in_features && a->x_sr % 4 == 0, "linear_f32: x row stride");
  const bool ln = a->ln_w != nullptr;
  SHRIMP_REQUIRE(!ln || a->ln_b, "linear_f32: ln_w without ln_b");
  const int64_t xe = (int64_t)(a->rows - 1) * a->x_sr + a->in_features;
  SHRIMP_REQUIRE(xe * 4 < (int64_t)0x7FFF0000, "linear_f32: activation buffer too large");
  Gemm32 g{};
  g.x = static_cast<const float*>(a->x);
  g.x_sb = a->x_sr;
  g.x_sr = a->x_sr;
  g.x_bytes = (uint32_t)(xe * 4);
  g.mask = a->mask;
  g.w = static_cast<const float*>(a->w);
  g.bias = a->bias;
  g.ln_w = a->ln_w;
  g.ln_b = a->ln_b;
  g.eps = a->eps;
  g.resid = static_cast<const float*>(a->resid);
  g.r_sb = a->r_sr;
  g.r_sr = a->r_sr;
  g.gamma = a->gamma;
  g.out = static_cast<float*>(a->out);
  g.o_sb = a->o_sr;
  g.o_sr = a->o_sr;
  g.B = a->rows;
  g.N = 1;
  g.kin = a->in_features;
  g.cout = a->out_features;
  g.S = a->S;
  g.H = a->H;
  g.dpad = a->dpad;
  hipStream_t st = as_stream(stream);
  switch (a->mode) {
    case SHRIMP_LIN_PLAIN:
      SHRIMP_REQUIRE(a->o_sr % 4 == 0, "linear_f32: out row stride %% 4");
      return ln ? dispatch_split<G_PLN>(g, st) : dispatch_split<0>(g, st);
    case SHRIMP_LIN_GELU:
      SHRIMP_REQUIRE(a->o_sr % 4 == 0, "linear_f32: out row stride %% 4");
      return ln ? dispatch_split<G_PLN | G_GELU>(g, st) : dispatch_split<G_GELU>(g, st);
    case SHRIMP_LIN_RESID:
      SHRIMP_REQUIRE(a->resid && a->gamma, "linear_f32: residual mode needs resid and gamma");
      SHRIMP_REQUIRE(!ln, "linear_f32: residual mode takes no LayerNorm prologue");
      SHRIMP_REQUIRE(a->o_sr % 4 == 0 && a->r_sr % 4 == 0, "linear_f32: row strides %% 4");
      return dispatch_split<G_LRES>(g, st);
    case SHRIMP_LIN_QKV:
      SHRIMP_REQUIRE(a->out_features % 3 == 0, "linear_f32: qkv out_features %% 3");
      SHRIMP_REQUIRE(a->B > 0 && a->S > 0 && a->H > 0 && (int64_t)a->B * a->S == a->rows,
                     "linear_f32: qkv needs B*S == rows");
      SHRIMP_REQUIRE((a->out_features / 3) % a->H == 0, "linear_f32: qkv C %% H != 0");
      SHRIMP_REQUIRE(((a->out_features / 3) / a->H) % 4 == 0 &&
                         a->dpad >= (a->out_features / 3) / a->H && a->dpad % 4 == 0,
                     "linear_f32: qkv head split needs d %% 4 == 0 and dpad >= d, dpad %% 4 == 0");
      return ln ? dispatch_split<G_PLN | G_QKV>(g, st) : dispatch_split<G_QKV>(g, st);
    default:
      return set_error(SHRIMP_EINVAL, "linear_f32: unknown mode %d", a->mode);
  }
}

extern "C" int shrimp_attn_f32(const shrimp_attn_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_f32: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->S > 0 && a->S <= kMaxDim && a->H > 0 && a->H <= kMaxDim,
                 "attn_f32: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  int npos = 0;
  if (int rc = check_attn_rows(a, 4, &npos)) return rc;
  hipStream_t st = as_stream(stream);
  // head dim 16 in coords mode: the MFMA kernel (variant 3 keeps the chunked
  // kernel, for comparison)
  const auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const size_t lds = attn32_mfma_lds(a->S);
  if (!a->pair && a->d == 16 && a->dpad == 16 && a->lut_m <= A32_XD && g_attn_variant != 3 &&
      lds <= (size_t)max_lds_per_block() && al16(a->q) && al16(a->k) && al16(a->v) && al16(a->o) &&
      a->qkv_sb % 4 == 0 && a->qkv_sh % 4 == 0 && a->o_sb % 4 == 0 && a->o_sh % 4 == 0 &&
      a->o_sr % 4 == 0) {
    hipLaunchKernelGGL(attn32_mfma_kernel, dim3(a->H, a->B), dim3(A32_NW * 64), lds, st, *a,
                       SHRIMP_LOG2E_F32 / sqrtf((float)a->d));
    return check_launch("attn32_mfma");
  }
  return a->pair ? launch_attn_rows<float, true>(a, npos, st)
                 : launch_attn_rows<float, false>(a, npos, st);
}

extern "C" int shrimp_prep_feats_f32(const void* feats, int feats_dt, int nfeat, int B, int N,
                                     float* xin, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && N > 0 && N <= kMaxDim, "prep_feats_f32: bad shape");
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(feats && xin && nfeat > 0 && nfeat <= 16, "prep_feats_f32: feats (nfeat %d)",
                 nfeat);
  const int64_t total = (int64_t)B * N * 16;
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t st = as_stream(stream);
  if (feats_dt == SHRIMP_DT_F32)
    hipLaunchKernelGGL(feats32_kernel<SHRIMP_DT_F32>, grid, dim3(256), 0, st, feats, nfeat, total, xin);
  else if (feats_dt == SHRIMP_DT_F16)
    hipLaunchKernelGGL(feats32_kernel<SHRIMP_DT_F16>, grid, dim3(256), 0, st, feats, nfeat, total, xin);
  else if (feats_dt == SHRIMP_DT_BF16)
    hipLaunchKernelGGL(feats32_kernel<SHRIMP_DT_BF16>, grid, dim3(256), 0, st, feats, nfeat, total, xin);
  else
    return set_error(SHRIMP_EINVAL, "prep_feats_f32: feats dtype %d", feats_dt);
  return check_launch("prep_feats_f32");
}

extern "C" int shrimp_prep_csr_feats_f32(const void* node_feats, int nfeat,
                                         const int64_t* row_offsets, int row0, int B, int N,
                                         float* xin, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && N > 0 && N <= kMaxDim && row0 >= 0, "prep_csr_feats_f32: bad sizes");
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(node_feats && row_offsets && xin && nfeat > 0 && nfeat <= 16,
                 "prep_csr_feats_f32: null pointer or nfeat %d", nfeat);
  hipLaunchKernelGGL(csr_feats32_kernel, dim3(4, B), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(node_feats), nfeat, row_offsets, row0, N, xin);
  return check_launch("prep_csr_feats_f32");
}

extern "C" int shrimp_fill_tokens_f32(const float* tokens, int n_tokens, int C, float* seq,
                                      int64_t seq_sb, int B, void* stream) {
  SHRIMP_REQUIRE(tokens && seq, "fill_tokens_f32: null pointer");
  if (B == 0 || n_tokens == 0) return SHRIMP_OK;
  hipLaunchKernelGGL(fill_tokens32_kernel, dim3(B), dim3(256), 0, as_stream(stream), tokens,
                     n_tokens * C, seq, seq_sb);
  return check_launch("fill_tokens_f32");
}
