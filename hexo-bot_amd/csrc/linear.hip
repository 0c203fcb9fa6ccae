// Dense row GEMM (nn.Linear) for gfx950 with fused LayerNorm prologue and
// GELU / residual / head-split epilogues: the projections and MLP of the
// attention block (packages/shrimp/python/shrimp/model.py:448-514).
//
// A wave owns MB x 16 rows; its whole K-slice of activations is loaded once
// into registers as MFMA B fragments (so the LayerNorm prologue normalises in
// registers), then the wave walks NW blocks of 16 outputs, streaming packed
// weight fragments (prefetched one block ahead). The product is computed
// transposed (out^T = W . x^T) on v_mfma_f32_16x16x32_bf16, so each lane ends
// with 4 adjacent outputs of one row and stores 8 bytes.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

template <int K, int MB, int NW, int MODE, bool LN>
__global__ __launch_bounds__(256, 2) void linear_kernel(const shrimp_linear_args a,
                                                        uint32_t x_bytes, uint32_t w_bytes) {
  constexpr int KS = K / 32;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int row_base = (blockIdx.x * 4 + wave) * (MB * 16);
  if (row_base >= a.rows) return;
  const int nbt = a.out_features >> 4;
  const int nb0 = blockIdx.y * NW;

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);

  u32x4 xa[MB][KS];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = row_base + mb * 16 + lr;
    const uint32_t base =
        r < a.rows ? (uint32_t)((int64_t)r * a.x_sr * 2) + (uint32_t)(lg * 16) : SHRIMP_OOB_OFFSET;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) xa[mb][ks] = buf_load16(xr, base + ks * 64);
  }

  if (LN) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float s = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) s += bf16_lo(xa[mb][ks][w]) + bf16_hi(xa[mb][ks][w]);
      const float mean = sum_lane_groups(s) * (1.0f / K);
      float q = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float u0 = bf16_lo(xa[mb][ks][w]) - mean;
          const float u1 = bf16_hi(xa[mb][ks][w]) - mean;
          q += u0 * u0 + u1 * u1;
        }
      const float rstd = rsqrtf(sum_lane_groups(q) * (1.0f / K) + a.eps);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int k0 = ks * 32 + lg * 8;
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(a.ln_w + k0);
        const f32x4 g1 = *reinterpret_cast<const f32x4*>(a.ln_w + k0 + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(a.ln_b + k0);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(a.ln_b + k0 + 4);
        const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        const float bb[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float u0 = (bf16_lo(xa[mb][ks][w]) - mean) * rstd * g[2 * w] + bb[2 * w];
          const float u1 = (bf16_hi(xa[mb][ks][w]) - mean) * rstd * g[2 * w + 1] + bb[2 * w + 1];
          xa[mb][ks][w] = pack_bf16x2(u0, u1);
        }
      }
    }
  }

  f32x4 acc[NW][MB];
#pragma unroll
  for (int nw = 0; nw < NW; ++nw)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nw][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 wn[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    wn[ks] = buf_load16(wr, (uint32_t)(((ks * nbt + nb0) * 64 + lane) * 16));
#pragma unroll
  for (int nw = 0; nw < NW; ++nw) {
    u32x4 wc[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) wc[ks] = wn[ks];
    if (nw + 1 < NW) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        wn[ks] = buf_load16(wr, (uint32_t)(((ks * nbt + nb0 + nw + 1) * 64 + lane) * 16));
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[nw][mb] = mfma16x16x32(wc[ks], xa[mb][ks], acc[nw][mb]);
  }

  // ---- epilogue ------------------------------------------------------------
  const int C3 = a.out_features / 3;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = row_base + mb * 16 + lr;
    if (r >= a.rows) continue;
    float live = 1.f;
    if (MODE == SHRIMP_LIN_RESID && a.mask != nullptr) live = a.mask[r] ? 1.f : 0.f;
    int bq = 0, sq = 0;
    if (MODE == SHRIMP_LIN_QKV) {
      bq = r / a.S;
      sq = r - bq * a.S;
    }
#pragma unroll
    for (int nw = 0; nw < NW; ++nw) {
      const int n = (nb0 + nw) * 16 + lg * 4;
      const f32x4 bb = *reinterpret_cast<const f32x4*>(a.bias + n);
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = acc[nw][mb][j] + bb[j];
      unsigned short* dst;
      if (MODE == SHRIMP_LIN_GELU) {
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = gelu_erf(o[j]);
      }
      unsigned short* lo_p = nullptr;  // this row's token low part (RESID mode)
      if (MODE == SHRIMP_LIN_RESID) {
        const u32x2 rw = *reinterpret_cast<const u32x2*>(
            static_cast<const unsigned short*>(a.resid) + (int64_t)r * a.r_sr + n);
        u32x2 lw = u32x2{0u, 0u};
        if (a.tok_lo != nullptr) {
          const int bp = r / a.S, sp = r - bp * a.S;
          if (sp < a.n_tokens) {
            lo_p = static_cast<unsigned short*>(a.tok_lo) +
                   ((int64_t)bp * a.n_tokens + sp) * a.out_features + n;
            lw = *reinterpret_cast<const u32x2*>(lo_p);
          }
        }
        const f32x4 g = *reinterpret_cast<const f32x4*>(a.gamma + n);
        o[0] = (bf16_lo(rw.x) + bf16_lo(lw.x)) + g[0] * (live * o[0]);
        o[1] = (bf16_hi(rw.x) + bf16_hi(lw.x)) + g[1] * (live * o[1]);
        o[2] = (bf16_lo(rw.y) + bf16_lo(lw.y)) + g[2] * (live * o[2]);
        o[3] = (bf16_hi(rw.y) + bf16_hi(lw.y)) + g[3] * (live * o[3]);
      }
      if (MODE == SHRIMP_LIN_QKV) {
        const int which = n / C3;
        const int nn = n - which * C3;
        const int dh = C3 / a.H;
        const int hh = nn / dh;
        const int dd = nn - hh * dh;
        dst = static_cast<unsigned short*>(a.out) +
              ((((int64_t)which * a.B + bq) * a.H + hh) * a.S + sq) * a.dpad + dd;
      } else {
        dst = static_cast<unsigned short*>(a.out) + (int64_t)r * a.o_sr + n;
      }
      u32x2 pk;
      pk.x = pack_bf16x2(o[0], o[1]);
      pk.y = pack_bf16x2(o[2], o[3]);
      *reinterpret_cast<u32x2*>(dst) = pk;
      if (MODE == SHRIMP_LIN_RESID && lo_p != nullptr) {
        *reinterpret_cast<u32x2*>(lo_p) =
            u32x2{pack_bf16x2(o[0] - bf16_lo(pk.x), o[1] - bf16_hi(pk.x)),
                  pack_bf16x2(o[2] - bf16_lo(pk.y), o[3] - bf16_hi(pk.y))};
      }
    }
  }
}

template <int K, int MB, int NW, int MODE, bool LN>
static int launch_linear(const shrimp_linear_args* a, uint32_t xb, uint32_t wb, hipStream_t st) {
  const int per_block = 4 * MB * 16;
  dim3 grid((a->rows + per_block - 1) / per_block, (a->out_features / 16) / NW);
  hipLaunchKernelGGL((linear_kernel<K, MB, NW, MODE, LN>), grid, dim3(256), 0, st, *a, xb, wb);
  return check_launch("linear");
}

template <int MODE, bool LN>
static int dispatch_k(const shrimp_linear_args* a, uint32_t xb, uint32_t wb, hipStream_t st) {
  const bool wide = ((a->out_features / 16) % 8) == 0;
#define SHRIMP_LIN_CASE(KK, MBB)                                                       \
  case KK:                                                                            \
    return wide ? launch_linear<KK, MBB, 8, MODE, LN>(a, xb, wb, st)                  \
                : launch_linear<KK, MBB, 2, MODE, LN>(a, xb, wb, st);
  switch (a->in_features) {
    SHRIMP_LIN_CASE(32, 4)
    SHRIMP_LIN_CASE(64, 4)
    SHRIMP_LIN_CASE(96, 4)
    SHRIMP_LIN_CASE(128, 4)
    SHRIMP_LIN_CASE(192, 2)
    SHRIMP_LIN_CASE(256, 2)
    SHRIMP_LIN_CASE(384, 1)
    default:
      return set_error(SHRIMP_EINVAL, "linear: unsupported in_features %d", a->in_features);
  }
#undef SHRIMP_LIN_CASE
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_linear(const shrimp_linear_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "linear: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "linear: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->w && a->bias && a->out, "linear: null pointer");
  SHRIMP_REQUIRE(a->out_features % 32 == 0, "linear: out_features %d %% 32 != 0",
                 a->out_features);
  SHRIMP_REQUIRE(strides_ok({a->x_sr, a->o_sr, a->r_sr}), "linear: row strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->x_sr >= a->in_features && a->x_sr % 8 == 0, "linear: x row stride");
  const bool ln = a->ln_w != nullptr;
  SHRIMP_REQUIRE(!ln || a->ln_b, "linear: ln_w without ln_b");
  const int64_t x_extent = (int64_t)(a->rows - 1) * a->x_sr + a->in_features;
  SHRIMP_REQUIRE(x_extent * 2 < (int64_t)0x7FFF0000, "linear: activation buffer too large");
  const uint32_t xb = (uint32_t)(x_extent * 2);
  const uint32_t wb = (uint32_t)shrimp_linear_wpack_bytes(a->in_features, a->out_features);
  hipStream_t st = as_stream(stream);
  switch (a->mode) {
    case SHRIMP_LIN_PLAIN:
      SHRIMP_REQUIRE(a->o_sr % 4 == 0, "linear: out row stride %% 4");
      return ln ? dispatch_k<SHRIMP_LIN_PLAIN, true>(a, xb, wb, st)
                : dispatch_k<SHRIMP_LIN_PLAIN, false>(a, xb, wb, st);
    case SHRIMP_LIN_GELU:
      SHRIMP_REQUIRE(a->o_sr % 4 == 0, "linear: out row stride %% 4");
      return ln ? dispatch_k<SHRIMP_LIN_GELU, true>(a, xb, wb, st)
                : dispatch_k<SHRIMP_LIN_GELU, false>(a, xb, wb, st);
    case SHRIMP_LIN_RESID:
      SHRIMP_REQUIRE(a->resid && a->gamma, "linear: residual mode needs resid and gamma");
      SHRIMP_REQUIRE(!ln, "linear: residual mode takes no LayerNorm prologue");
      SHRIMP_REQUIRE(a->o_sr % 4 == 0 && a->r_sr % 4 == 0, "linear: row strides %% 4");
      SHRIMP_REQUIRE(!a->tok_lo || (a->S > 0 && a->rows % a->S == 0 && a->n_tokens >= 0 &&
                                    a->n_tokens <= a->S),
                     "linear: token low parts need rows = whole positions of S rows");
      return dispatch_k<SHRIMP_LIN_RESID, false>(a, xb, wb, st);
    case SHRIMP_LIN_QKV:
      SHRIMP_REQUIRE(a->out_features % 3 == 0, "linear: qkv out_features %% 3");
      SHRIMP_REQUIRE(a->B > 0 && a->S > 0 && a->H > 0 && (int64_t)a->B * a->S == a->rows,
                     "linear: qkv needs B*S == rows");
      SHRIMP_REQUIRE((a->out_features / 3) % a->H == 0, "linear: qkv C %% H != 0");
      SHRIMP_REQUIRE(((a->out_features / 3) / a->H) % 4 == 0 &&
                         a->dpad >= (a->out_features / 3) / a->H && a->dpad % 16 == 0,
                     "linear: qkv head split needs d %% 4 == 0 and dpad >= d, dpad %% 16 == 0");
      return ln ? dispatch_k<SHRIMP_LIN_QKV, true>(a, xb, wb, st)
                : dispatch_k<SHRIMP_LIN_QKV, false>(a, xb, wb, st);
    default:
      return set_error(SHRIMP_EINVAL, "linear: unknown mode %d", a->mode);
  }
}
