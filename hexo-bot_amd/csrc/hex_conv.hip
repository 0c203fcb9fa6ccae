// Gather-GEMM hex / ray-tap convolution for gfx950 with fused epilogues.
//
// Semantics: HexNodeConv.forward (packages/shrimp/python/shrimp/model.py:346-370)
// with the epilogues of hex_conv_ln (_triton_conv.py:139-196), ConvBlock
// (model.py:395-422) and the policy head (model.py:1011-1020). The ray-tap op
// is the same kernel with 31 taps and a 32-slot index.
//
// Work split: a workgroup is 4 waves; each wave owns MB x 16 output rows and
// all COUT output channels, so LayerNorm over channels stays inside the wave.
// The product is computed transposed, out^T = W^T . X^T, on
// v_mfma_f32_16x16x32_bf16:
//   A operand = packed weight fragment (16 couts x 32 k), one 16-byte load;
//   B operand = gathered activation fragment (32 k x 16 rows): lane l reads
//               16 contiguous bytes of row idx[row(l%16), t] -> one buffer load
//               per lane, rows outside [0, N) come back as zeros;
//   result    = lane l holds couts 4*(l/16)+j of row l%16, so each lane stores
//               4 adjacent bf16 (8 bytes) and LayerNorm reduces over the four
//               lane groups with two cross-lane steps.
// Next k-step fragments are loaded before the current step's MFMAs issue, so
// the gather latency overlaps the matrix work of the previous step.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

enum : int { EPI_LN = 1, EPI_RELU = 2, EPI_RESID = 4, EPI_HEAD = 8 };

template <int COUT, int MB, int EPI>
__global__ __launch_bounds__(256, 2) void hex_conv_kernel(const shrimp_conv_args a,
                                                          uint32_t x_bytes, uint32_t w_bytes) {
  constexpr int NB = COUT / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int N = a.N;
  const int total = a.B * N;
  const int row_base = (blockIdx.x * 4 + wave) * (MB * 16);
  if (row_base >= total) return;

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);

  int rb[MB], rn[MB];
  bool rv[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = row_base + mb * 16 + lr;
    rv[mb] = r < total;
    rb[mb] = rv[mb] ? r / N : 0;
    rn[mb] = rv[mb] ? r - rb[mb] * N : 0;
  }

  const int kc_n = a.cin_pad >> 5;
  const int nsteps = a.taps * kc_n;

  // Byte offset (k-slice of this lane included) of the gathered row for tap t.
  auto tap_offsets = [&](int t, uint32_t (&off)[MB]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      int j = -1;
      if (rv[mb]) j = a.idx[(int64_t)(rb[mb] * N + rn[mb]) * a.idx_stride + t];
      const bool ok = (j >= 0) && (j < N);
      const int64_t e = (int64_t)rb[mb] * a.x_sb + (int64_t)j * a.x_sn;
      off[mb] = ok ? (uint32_t)(e * 2) + (uint32_t)(lg * 16) : SHRIMP_OOB_OFFSET;
    }
  };

  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint32_t off[MB];
  tap_offsets(0, off);
  u32x4 xf[MB], wf[NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xf[mb] = buf_load16(xr, off[mb]);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) wf[nb] = buf_load16(wr, (uint32_t)((nb * 64 + lane) * 16));

  int t = 0, kc = 0;
  for (int s = 0; s < nsteps; ++s) {
    u32x4 xc[MB], wc[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xc[mb] = xf[mb];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) wc[nb] = wf[nb];
    if (s + 1 < nsteps) {
      if (++kc == kc_n) {
        kc = 0;
        ++t;
        tap_offsets(t, off);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) xf[mb] = buf_load16(xr, off[mb] + (uint32_t)(kc * 64));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        wf[nb] = buf_load16(wr, (uint32_t)((((s + 1) * NB + nb) * 64 + lane) * 16));
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma16x16x32(wc[nb], xc[mb], acc[nb][mb]);
  }

  // ---- epilogue ------------------------------------------------------------
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float v[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 bb = *reinterpret_cast<const f32x4*>(a.bias + nb * 16 + lg * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[nb][j] = acc[nb][mb][j] + bb[j];
    }
    if (EPI & EPI_LN) {
      float s = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += v[nb][j];
      const float mean = sum_lane_groups(s) * (1.0f / COUT);
      float q = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[nb][j] -= mean;
          q += v[nb][j] * v[nb][j];
        }
      const float rstd = rsqrtf(sum_lane_groups(q) * (1.0f / COUT) + a.eps);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 gw = *reinterpret_cast<const f32x4*>(a.ln_w + nb * 16 + lg * 4);
        const f32x4 gb = *reinterpret_cast<const f32x4*>(a.ln_b + nb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[nb][j] = v[nb][j] * rstd * gw[j] + gb[j];
      }
    }
    if (EPI & EPI_RELU) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[nb][j] = fmaxf(v[nb][j], 0.f);
    }
    const bool live = rv[mb] && a.mask[(int64_t)rb[mb] * N + rn[mb]] != 0;
    if (EPI & EPI_HEAD) {
      float h = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 hw = *reinterpret_cast<const f32x4*>(a.head_w + nb * 16 + lg * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) h += v[nb][j] * hw[j];
      }
      h = sum_lane_groups(h);
      if (rv[mb] && lg == 0) a.head_out[(int64_t)rb[mb] * N + rn[mb]] = live ? h + a.head_b[0] : 0.f;
      continue;
    }
    if (!rv[mb]) continue;
    const int64_t obase = (int64_t)rb[mb] * a.o_sb + (int64_t)rn[mb] * a.o_sn + lg * 4;
    const int64_t rbase = (int64_t)rb[mb] * a.r_sb + (int64_t)rn[mb] * a.r_sn + lg * 4;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = live ? v[nb][j] : 0.f;
      if (EPI & EPI_RESID) {
        const u32x2 rw =
            *reinterpret_cast<const u32x2*>(static_cast<const unsigned short*>(a.resid) + rbase + nb * 16);
        const f32x4 g = *reinterpret_cast<const f32x4*>(a.gamma + nb * 16 + lg * 4);
        o[0] = fmaxf(bf16_lo(rw.x) + g[0] * o[0], 0.f);
        o[1] = fmaxf(bf16_hi(rw.x) + g[1] * o[1], 0.f);
        o[2] = fmaxf(bf16_lo(rw.y) + g[2] * o[2], 0.f);
        o[3] = fmaxf(bf16_hi(rw.y) + g[3] * o[3], 0.f);
      }
      u32x2 pk;
      pk.x = pack_bf16x2(o[0], o[1]);
      pk.y = pack_bf16x2(o[2], o[3]);
      *reinterpret_cast<u32x2*>(static_cast<unsigned short*>(a.out) + obase + nb * 16) = pk;
    }
  }
}

// ---- weight packing ------------------------------------------------------------
// Fragment f = (ks * NB + nb) * 64 + lane holds 8 bf16:
//   W[k = 32*ks + 8*(lane/16) + e][n = 16*nb + lane%16],  k = t*cin_pad + c.
__global__ void pack_weight_kernel(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                   int K, int NOUT, int cin, int cin_pad, int64_t s_t,
                                   int64_t s_c, int64_t s_n) {
  const int NB = NOUT / 16;
  const int64_t frags = (int64_t)(K / 32) * NB * 64;
  const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= frags) return;
  const int lane = (int)(f & 63);
  const int nb = (int)((f >> 6) % NB);
  const int ks = (int)((f >> 6) / NB);
  const int n = nb * 16 + (lane & 15);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = ks * 32 + (lane >> 4) * 8 + e;
    const int t = k / cin_pad;
    const int c = k - t * cin_pad;
    const float v = (c < cin) ? src[t * s_t + c * s_c + n * s_n] : 0.f;
    dst[f * 8 + e] = f32_to_bf16_bits(v);
  }
}

template <int COUT, int MB, int EPI>
static int launch_conv(const shrimp_conv_args* a, uint32_t xb, uint32_t wb, hipStream_t st) {
  const int rows = a->B * a->N;
  const int per_block = 4 * MB * 16;
  const int grid = (rows + per_block - 1) / per_block;
  hipLaunchKernelGGL((hex_conv_kernel<COUT, MB, EPI>), dim3(grid), dim3(256), 0, st, *a, xb, wb);
  return check_launch("hex_conv");
}

template <int EPI>
static int dispatch_cout(const shrimp_conv_args* a, uint32_t xb, uint32_t wb, hipStream_t st) {
  switch (a->cout) {
    case 32: return launch_conv<32, 4, EPI>(a, xb, wb, st);
    case 64: return launch_conv<64, 4, EPI>(a, xb, wb, st);
    case 96: return launch_conv<96, 4, EPI>(a, xb, wb, st);
    case 128: return launch_conv<128, 4, EPI>(a, xb, wb, st);
    case 192: return launch_conv<192, 2, EPI>(a, xb, wb, st);
    case 256: return launch_conv<256, 1, EPI>(a, xb, wb, st);
    default: return set_error(SHRIMP_EINVAL, "hex_conv: unsupported cout %d", a->cout);
  }
}

}  // namespace shrimp

using namespace shrimp;

extern "C" size_t shrimp_conv_wpack_bytes(int taps, int cin_pad, int cout) {
  return (size_t)taps * cin_pad * cout * 2;
}

extern "C" size_t shrimp_linear_wpack_bytes(int in_features, int out_features) {
  return (size_t)in_features * out_features * 2;
}

extern "C" int shrimp_pack_conv_weight(const float* w, void* packed, int taps, int cin,
                                       int cin_pad, int cout, void* stream) {
  SHRIMP_REQUIRE(w && packed, "pack_conv_weight: null pointer");
  SHRIMP_REQUIRE(taps > 0 && cin > 0 && cin <= cin_pad && cin_pad % 32 == 0,
                 "pack_conv_weight: bad taps/cin (%d, %d, %d)", taps, cin, cin_pad);
  SHRIMP_REQUIRE(cout > 0 && cout % 16 == 0, "pack_conv_weight: cout %d not a multiple of 16",
                 cout);
  const int K = taps * cin_pad;
  const int64_t frags = (int64_t)(K / 32) * (cout / 16) * 64;
  const int grid = (int)((frags + 255) / 256);
  hipLaunchKernelGGL(pack_weight_kernel, dim3(grid), dim3(256), 0, as_stream(stream), w,
                     static_cast<unsigned short*>(packed), K, cout, cin, cin_pad,
                     (int64_t)cin * cout, (int64_t)cout, (int64_t)1);
  return check_launch("pack_conv_weight");
}

extern "C" int shrimp_pack_linear_weight(const float* w, void* packed, int in_features,
                                         int out_features, void* stream) {
  SHRIMP_REQUIRE(w && packed, "pack_linear_weight: null pointer");
  SHRIMP_REQUIRE(in_features % 32 == 0 && out_features % 16 == 0,
                 "pack_linear_weight: shape (%d -> %d) needs in %% 32 == 0, out %% 16 == 0",
                 in_features, out_features);
  const int64_t frags = (int64_t)(in_features / 32) * (out_features / 16) * 64;
  const int grid = (int)((frags + 255) / 256);
  hipLaunchKernelGGL(pack_weight_kernel, dim3(grid), dim3(256), 0, as_stream(stream), w,
                     static_cast<unsigned short*>(packed), in_features, out_features,
                     in_features, in_features, (int64_t)0, (int64_t)1, (int64_t)in_features);
  return check_launch("pack_linear_weight");
}

extern "C" int shrimp_hex_conv(const shrimp_conv_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "hex_conv: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->N > 0, "hex_conv: bad B/N (%d, %d)", a->B, a->N);
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->idx && a->mask && a->w && a->bias, "hex_conv: null input pointer");
  SHRIMP_REQUIRE(a->taps > 0 && a->idx_stride >= a->taps, "hex_conv: bad taps %d / stride %d",
                 a->taps, a->idx_stride);
  SHRIMP_REQUIRE(a->cin_pad > 0 && a->cin_pad % 32 == 0, "hex_conv: cin_pad %d %% 32 != 0",
                 a->cin_pad);
  SHRIMP_REQUIRE(a->x_sn >= a->cin_pad && a->x_sn % 8 == 0,
                 "hex_conv: row stride %lld must be >= cin_pad and a multiple of 8",
                 (long long)a->x_sn);
  const bool head = a->head_w != nullptr;
  const bool ln = a->ln_w != nullptr;
  const bool resid = a->resid != nullptr;
  SHRIMP_REQUIRE(!ln || a->ln_b, "hex_conv: ln_w without ln_b");
  SHRIMP_REQUIRE(!resid || a->gamma, "hex_conv: residual needs gamma");
  SHRIMP_REQUIRE(head ? (a->head_out != nullptr && a->head_b != nullptr) : (a->out != nullptr),
                 "hex_conv: no output");
  SHRIMP_REQUIRE(!head || (!ln && !resid), "hex_conv: head epilogue excludes LN / residual");
  if (!head) {
    SHRIMP_REQUIRE(a->o_sn % 4 == 0 && a->o_sb % 4 == 0, "hex_conv: output strides %% 4");
    SHRIMP_REQUIRE(!resid || (a->r_sn % 4 == 0 && a->r_sb % 4 == 0),
                   "hex_conv: residual strides %% 4");
  }
  const int64_t x_extent = (int64_t)(a->B - 1) * a->x_sb + (int64_t)(a->N - 1) * a->x_sn + a->cin_pad;
  SHRIMP_REQUIRE(x_extent * 2 < (int64_t)0x7FFF0000, "hex_conv: activation buffer too large");
  const uint32_t xb = (uint32_t)(x_extent * 2);
  const uint32_t wb = (uint32_t)shrimp_conv_wpack_bytes(a->taps, a->cin_pad, a->cout);
  hipStream_t st = as_stream(stream);
  if (head) {
    SHRIMP_REQUIRE(a->relu, "hex_conv: head epilogue expects relu");
    return dispatch_cout<EPI_HEAD | EPI_RELU>(a, xb, wb, st);
  }
  if (resid) {
    SHRIMP_REQUIRE(ln && !a->relu, "hex_conv: residual epilogue is LN (no relu) + residual");
    return dispatch_cout<EPI_LN | EPI_RESID>(a, xb, wb, st);
  }
  if (ln) {
    return a->relu ? dispatch_cout<EPI_LN | EPI_RELU>(a, xb, wb, st)
                   : dispatch_cout<EPI_LN>(a, xb, wb, st);
  }
  return a->relu ? dispatch_cout<EPI_RELU>(a, xb, wb, st) : dispatch_cout<0>(a, xb, wb, st);
}
