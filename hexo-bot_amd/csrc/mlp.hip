// Fused tail of the attention block for gfx950 (AttnBlock.forward after the
// attention core, packages/shrimp/python/shrimp/model.py:508-514):
//
//   s1  = seq + g_attn * (m * (att . Wo^T + bo))          (out_proj, LayerScale)
//   h   = GELU_erf(LN2(s1) . W1^T + b1)                   (fc1, hidden 2C)
//   seq = s1 + g_mlp * (m * (h . W2^T + b2))              (fc2, LayerScale)
//
// with s1 and h rounded to bf16 where the unfused kernels store them.
//
// Layout: one persistent workgroup per CU keeps the three packed weight
// matrices in LDS (C = 128: 32 + 64 + 64 KiB = the whole 160 KiB), and each
// of its 8 waves streams blocks of 16 rows through the three products without
// leaving registers: a product's output fragment (lane l: channels
// 16 nb + 4 (l/16) + j of row l % 16) is directly the next product's input
// fragment for K-step ks = nb / 2, because fc1 and fc2 are packed with that
// interleaved K order (shrimp_pack_linear_weight_il). Only att and seq touch
// HBM: 3 x 256 bytes per row.
#include <algorithm>

#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

namespace {

constexpr int MC = 128;           // channels
constexpr int MH = 2 * MC;        // hidden width
constexpr int MWAVES = 8;         // waves per workgroup (2 per SIMD)
constexpr uint32_t WO_OFF = 0;                        // out_proj fragments
constexpr uint32_t W1_OFF = MC * MC * 2;              // fc1 fragments
constexpr uint32_t W2_OFF = W1_OFF + MC * MH * 2;     // fc2 fragments
constexpr uint32_t W_LDS = W2_OFF + MH * MC * 2;      // 163840 bytes

// GELU with erf from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7 on erf):
//   erfc(z) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),
//   t = 1 / (1 + p z), z = |x| / sqrt(2) >= 0,
// GELU(x) = x * Phi(x), Phi(x) = 1 - erfc(z) / 2 for x >= 0, erfc(z) / 2 else.
SHRIMP_DEV float gelu_as(float x) {
  constexpr float p = 0.3275911f * 0.70710678118654752f;  // p / sqrt(2), applied to |x|
  constexpr float a1 = 0.5f * 0.254829592f, a2 = 0.5f * -0.284496736f, a3 = 0.5f * 1.421413741f;
  constexpr float a4 = 0.5f * -1.453152027f, a5 = 0.5f * 1.061405429f;
  constexpr float nh = -0.5f * 1.4426950408889634f;       // exp(-x^2/2) = exp2(nh * x^2)
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(p, ax, 1.0f));
  float q = fmaf(a5, t, a4);
  q = fmaf(q, t, a3);
  q = fmaf(q, t, a2);
  q = fmaf(q, t, a1);
  q *= t;                                                  // erfc(z) / 2 before the exp factor
  const float h = q * __builtin_amdgcn_exp2f(nh * (x * x));  // erfc(z) / 2
  const float phi = x >= 0.f ? 1.0f - h : h;
  return x * phi;
}

SHRIMP_DEV u32x4 lds_frag(const unsigned char* wl, uint32_t base, int ks, int nb, int nbt,
                          int lane) {
  return *reinterpret_cast<const u32x4*>(wl + base + (uint32_t)(((ks * nbt + nb) * 64 + lane) * 16));
}

template <int MB>
SHRIMP_DEV void mlp_rows(const shrimp_mlp_args& a, const unsigned char* wl,
                         __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t sr, int row0,
                         int lane) {
  constexpr int KS1 = MC / 32, NB1 = MC / 16, NBH = MH / 16, KT = MH / 32, NB2 = MC / 16;
  const int lr = lane & 15, lg = lane >> 4;
  const float* __restrict__ ob = a.out_b;
  const float* __restrict__ ga = a.g_attn;
  const float* __restrict__ lw = a.ln_w;
  const float* __restrict__ lb = a.ln_b;
  const float* __restrict__ b1 = a.fc1_b;
  const float* __restrict__ b2 = a.fc2_b;
  const float* __restrict__ gm = a.g_mlp;

  int r[MB];
  bool rv[MB];
  float live[MB];
  u32x4 xf[MB][KS1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    r[mb] = row0 + mb * 16 + lr;
    rv[mb] = r[mb] < a.rows;
    const uint32_t off = rv[mb] ? (uint32_t)((int64_t)r[mb] * a.x_sr * 2) + (uint32_t)(lg * 16)
                                : SHRIMP_OOB_OFFSET;
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) xf[mb][ks] = buf_load16(xr, off + ks * 64);
  }
  // residual rows (bf16, 4 channels per 16-channel block)
  u32x2 sp[MB][NB1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    live[mb] = (rv[mb] && a.mask[r[mb]] != 0) ? 1.f : 0.f;
    const uint32_t off = rv[mb] ? (uint32_t)((int64_t)r[mb] * a.s_sr * 2) + (uint32_t)(lg * 8)
                                : SHRIMP_OOB_OFFSET;
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb) sp[mb][nb] = buf_load8(sr, off + nb * 32);
  }

  // ---- out_proj ----------------------------------------------------------
  f32x4 acc[MB][NB1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // (scheduling barriers keep the weight-fragment reads next to their MFMAs;
  // hoisted all at once they would not fit in registers)
#pragma unroll
  for (int nb = 0; nb < NB1; ++nb) {
    u32x4 w[KS1];
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) w[ks] = lds_frag(wl, WO_OFF, ks, nb, NB1, lane);
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16x16x32(w[ks], xf[mb][ks], acc[mb][nb]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- residual 1 (bf16 s1), LayerNorm 2 -> fc1 input fragments ------------
  u32x4 hf[MB][KS1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float v[NB1][4];
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = nb * 16 + lg * 4;
      const f32x4 bb = *reinterpret_cast<const f32x4*>(ob + c);
      const f32x4 g = *reinterpret_cast<const f32x4*>(ga + c);
      const float o0 = bf16_lo(sp[mb][nb].x) + g[0] * (live[mb] * (acc[mb][nb][0] + bb[0]));
      const float o1 = bf16_hi(sp[mb][nb].x) + g[1] * (live[mb] * (acc[mb][nb][1] + bb[1]));
      const float o2 = bf16_lo(sp[mb][nb].y) + g[2] * (live[mb] * (acc[mb][nb][2] + bb[2]));
      const float o3 = bf16_hi(sp[mb][nb].y) + g[3] * (live[mb] * (acc[mb][nb][3] + bb[3]));
      sp[mb][nb].x = pack_bf16x2(o0, o1);
      sp[mb][nb].y = pack_bf16x2(o2, o3);
      v[nb][0] = bf16_lo(sp[mb][nb].x);
      v[nb][1] = bf16_hi(sp[mb][nb].x);
      v[nb][2] = bf16_lo(sp[mb][nb].y);
      v[nb][3] = bf16_hi(sp[mb][nb].y);
    }
    float s = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) s += v[nb][j];
    const float mean = sum_groups_swap(s) * (1.0f / MC);
    float q = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[nb][j] -= mean;
        q += v[nb][j] * v[nb][j];
      }
    const float rstd = rsqrtf(sum_groups_swap(q) * (1.0f / MC) + a.eps);
    unsigned hp[NB1][2];
#pragma unroll
    for (int nb = 0; nb < NB1; ++nb) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = nb * 16 + lg * 4;
      const f32x4 gw = *reinterpret_cast<const f32x4*>(lw + c);
      const f32x4 gb = *reinterpret_cast<const f32x4*>(lb + c);
      hp[nb][0] = pack_bf16x2(v[nb][0] * rstd * gw[0] + gb[0], v[nb][1] * rstd * gw[1] + gb[1]);
      hp[nb][1] = pack_bf16x2(v[nb][2] * rstd * gw[2] + gb[2], v[nb][3] * rstd * gw[3] + gb[3]);
    }
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks)
      hf[mb][ks] = u32x4{hp[2 * ks][0], hp[2 * ks][1], hp[2 * ks + 1][0], hp[2 * ks + 1][1]};
  }

  // ---- fc1 -> GELU -> fc2, one 32-wide hidden slice at a time ---------------
  f32x4 acc2[MB][NB2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB2; ++nb) acc2[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int kt = 0; kt < KT; ++kt) {
    f32x4 ah[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) ah[mb][0] = ah[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) {
        const u32x4 w = lds_frag(wl, W1_OFF, ks, 2 * kt + hh, NBH, lane);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) ah[mb][hh] = mfma16x16x32(w, hf[mb][ks], ah[mb][hh]);
      }
    const f32x4 bh0 = *reinterpret_cast<const f32x4*>(b1 + (2 * kt) * 16 + lg * 4);
    const f32x4 bh1 = *reinterpret_cast<const f32x4*>(b1 + (2 * kt + 1) * 16 + lg * 4);
    u32x4 gf[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      gf[mb][0] = pack_bf16x2(gelu_as(ah[mb][0][0] + bh0[0]), gelu_as(ah[mb][0][1] + bh0[1]));
      gf[mb][1] = pack_bf16x2(gelu_as(ah[mb][0][2] + bh0[2]), gelu_as(ah[mb][0][3] + bh0[3]));
      gf[mb][2] = pack_bf16x2(gelu_as(ah[mb][1][0] + bh1[0]), gelu_as(ah[mb][1][1] + bh1[1]));
      gf[mb][3] = pack_bf16x2(gelu_as(ah[mb][1][2] + bh1[2]), gelu_as(ah[mb][1][3] + bh1[3]));
    }
#pragma unroll
    for (int nb = 0; nb < NB2; ++nb) {
      const u32x4 w = lds_frag(wl, W2_OFF, kt, nb, NB2, lane);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc2[mb][nb] = mfma16x16x32(w, gf[mb], acc2[mb][nb]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- residual 2 -> seq ----------------------------------------------------
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (!rv[mb]) continue;
    unsigned short* op = static_cast<unsigned short*>(a.seq) + (int64_t)r[mb] * a.s_sr + lg * 4;
#pragma unroll
    for (int nb = 0; nb < NB2; ++nb) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = nb * 16 + lg * 4;
      const f32x4 bb = *reinterpret_cast<const f32x4*>(b2 + c);
      const f32x4 g = *reinterpret_cast<const f32x4*>(gm + c);
      const float o0 = bf16_lo(sp[mb][nb].x) + g[0] * (live[mb] * (acc2[mb][nb][0] + bb[0]));
      const float o1 = bf16_hi(sp[mb][nb].x) + g[1] * (live[mb] * (acc2[mb][nb][1] + bb[1]));
      const float o2 = bf16_lo(sp[mb][nb].y) + g[2] * (live[mb] * (acc2[mb][nb][2] + bb[2]));
      const float o3 = bf16_hi(sp[mb][nb].y) + g[3] * (live[mb] * (acc2[mb][nb][3] + bb[3]));
      u32x2 pk;
      pk.x = pack_bf16x2(o0, o1);
      pk.y = pack_bf16x2(o2, o3);
      *reinterpret_cast<u32x2*>(op + nb * 16) = pk;
    }
  }
}

}  // namespace

__global__ __launch_bounds__(MWAVES * 64, 1) void attn_mlp_kernel(const shrimp_mlp_args a,
                                                                  uint32_t x_bytes,
                                                                  uint32_t s_bytes) {
  extern __shared__ __attribute__((aligned(16))) unsigned char wl[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // All three weight matrices into LDS (16-byte chunks, fragment order kept).
  {
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.out_w, W1_OFF);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(a.fc1_w, W2_OFF - W1_OFF);
    const __amdgpu_buffer_rsrc_t r2 = make_rsrc(a.fc2_w, W_LDS - W2_OFF);
    constexpr int CHUNKS = W_LDS / 16;
    constexpr int PER = CHUNKS / (MWAVES * 64);
    static_assert(CHUNKS % (MWAVES * 64) == 0, "weight chunks must tile the workgroup");
    u32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t off = (uint32_t)(i * MWAVES * 64 + threadIdx.x) * 16;
      v[i] = off < W1_OFF ? buf_load16(r0, off)
                          : (off < W2_OFF ? buf_load16(r1, off - W1_OFF) : buf_load16(r2, off - W2_OFF));
    }
#pragma unroll
    for (int i = 0; i < PER; ++i)
      *reinterpret_cast<u32x4*>(wl + (uint32_t)(i * MWAVES * 64 + threadIdx.x) * 16) = v[i];
  }
  __syncthreads();

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.seq, s_bytes);
  // Contiguous, balanced range of 16-row blocks per wave.
  const int64_t nblk = (a.rows + 15) / 16;
  const int64_t tw = (int64_t)gridDim.x * MWAVES;
  const int64_t gw = (int64_t)blockIdx.x * MWAVES + wave;
  int blk = (int)(gw * nblk / tw);
  const int end = (int)((gw + 1) * nblk / tw);
  for (; blk + 2 <= end; blk += 2) mlp_rows<2>(a, wl, xr, sr, blk * 16, lane);
  if (blk < end) mlp_rows<1>(a, wl, xr, sr, blk * 16, lane);
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_attn_mlp(const shrimp_mlp_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_mlp: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "attn_mlp: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->C == MC && a->hidden == MH,
                 "attn_mlp: fused kernel covers C=%d, hidden=%d (got C=%d, hidden=%d)", MC, MH,
                 a->C, a->hidden);
  SHRIMP_REQUIRE(a->x && a->seq && a->mask && a->out_w && a->out_b && a->g_attn && a->ln_w &&
                     a->ln_b && a->fc1_w && a->fc1_b && a->fc2_w && a->fc2_b && a->g_mlp,
                 "attn_mlp: null pointer");
  SHRIMP_REQUIRE(a->x_sr >= MC && a->x_sr % 8 == 0 && a->s_sr >= MC && a->s_sr % 8 == 0,
                 "attn_mlp: row strides must be >= C and multiples of 8");
  const int64_t xe = ((int64_t)(a->rows - 1) * a->x_sr + MC) * 2;
  const int64_t se = ((int64_t)(a->rows - 1) * a->s_sr + MC) * 2;
  SHRIMP_REQUIRE(xe < (int64_t)0x7FFF0000 && se < (int64_t)0x7FFF0000,
                 "attn_mlp: activation buffer too large");
  SHRIMP_REQUIRE((size_t)max_lds_per_block() >= W_LDS,
                 "attn_mlp: needs %u bytes of LDS per workgroup", (unsigned)W_LDS);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return set_error(SHRIMP_ELAUNCH, "attn_mlp: cannot query the compute unit count");
  const int64_t nblk = (a->rows + 15) / 16;
  const int grid = (int)std::min<int64_t>(cus, (nblk + MWAVES - 1) / MWAVES);
  hipLaunchKernelGGL(attn_mlp_kernel, dim3(grid), dim3(MWAVES * 64), W_LDS, as_stream(stream), *a,
                     (uint32_t)xe, (uint32_t)se);
  return check_launch("attn_mlp");
}
