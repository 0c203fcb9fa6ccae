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

// Bias / LayerNorm / ReLU / mask / residual / head epilogue on the fp32
// accumulators of MB row blocks. rb, rn: position and cell index of this
// lane's row in block mb; rv: row exists.
// Per-channel parameters (PSRC): PS_GLOBAL reads them where used; PS_REGS
// loads this lane's channels once into registers (re-reading after a store
// would wait, since the compiler must assume the store may alias them);
// PS_LDS reads them from an LDS copy at `lp` laid out [bias | ln_w | ln_b |
// gamma or head_w], COUT floats each.
// The row masks are loaded up front and the residual rows of block mb+1 are
// requested before block mb's math.
enum : int { PS_GLOBAL = 0, PS_REGS = 1, PS_LDS = 2 };

template <int COUT, int MB, int EPI, int PSRC>
SHRIMP_DEV void conv_epilogue(const shrimp_conv_args& a, f32x4 (&acc)[COUT / 16][MB],
                              const int (&rb)[MB], const int (&rn)[MB], const bool (&rv)[MB],
                              int lg, const float* lp = nullptr) {
  constexpr int NB = COUT / 16;
  constexpr bool LN = (EPI & EPI_LN) != 0, RESID = (EPI & EPI_RESID) != 0;
  constexpr bool HEAD = (EPI & EPI_HEAD) != 0;
  constexpr bool PRE = PSRC == PS_REGS;
  constexpr int PN = PRE ? NB : 1;
  const int N = a.N;
  f32x4 pb[PN], pw[LN ? PN : 1], pl[LN ? PN : 1], pg[RESID ? PN : 1], ph[HEAD ? PN : 1];
  auto prm = [&](const float* p, int nb) { return *reinterpret_cast<const f32x4*>(p + nb * 16 + lg * 4); };
  if constexpr (PRE) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      pb[nb] = prm(a.bias, nb);
      if constexpr (LN) {
        pw[nb] = prm(a.ln_w, nb);
        pl[nb] = prm(a.ln_b, nb);
      }
      if constexpr (RESID) pg[nb] = prm(a.gamma, nb);
      if constexpr (HEAD) ph[nb] = prm(a.head_w, nb);
    }
  }
  // ri: index into the register copy (0 when that array is a placeholder)
  auto pick = [&](int slot, const float* g, const f32x4* r, int nb, int ri) -> f32x4 {
    if constexpr (PSRC == PS_LDS) return prm(lp + slot * COUT, nb);
    else if constexpr (PRE) return r[ri];
    else return prm(g, nb);
  };
  auto P_b = [&](int nb) { return pick(0, a.bias, pb, nb, nb); };
  auto P_w = [&](int nb) { return pick(1, a.ln_w, pw, nb, LN && PRE ? nb : 0); };
  auto P_l = [&](int nb) { return pick(2, a.ln_b, pl, nb, LN && PRE ? nb : 0); };
  auto P_g = [&](int nb) { return pick(3, a.gamma, pg, nb, RESID && PRE ? nb : 0); };
  auto P_h = [&](int nb) { return pick(3, a.head_w, ph, nb, HEAD && PRE ? nb : 0); };
  bool live[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) live[mb] = rv[mb] && a.mask[(int64_t)rb[mb] * N + rn[mb]] != 0;
  const float hb = HEAD ? a.head_b[0] : 0.f;

  auto resid_row = [&](int mb, u32x2 (&r)[NB]) {
    if constexpr (RESID) {
      const unsigned short* rp = static_cast<const unsigned short*>(a.resid) +
                                 (int64_t)rb[mb] * a.r_sb + (int64_t)rn[mb] * a.r_sn + lg * 4;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        r[nb] = rv[mb] ? *reinterpret_cast<const u32x2*>(rp + nb * 16) : u32x2{0u, 0u};
    }
  };
  u32x2 rcur[RESID ? NB : 1], rnext[RESID ? NB : 1];
  if constexpr (RESID) resid_row(0, rcur);

#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if constexpr (RESID) {
      if (mb + 1 < MB) resid_row(mb + 1, rnext);
    }
    float v[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 bb = P_b(nb);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[nb][j] = acc[nb][mb][j] + bb[j];
    }
    if constexpr (LN) {
      float s = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += v[nb][j];
      const float mean = sum_groups_swap(s) * (1.0f / COUT);
      float q = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[nb][j] -= mean;
          q += v[nb][j] * v[nb][j];
        }
      const float rstd = rsqrtf(sum_groups_swap(q) * (1.0f / COUT) + a.eps);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 gw = P_w(nb), gb = P_l(nb);
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
    if constexpr (HEAD) {
      float h = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 hw = P_h(nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) h += v[nb][j] * hw[j];
      }
      h = sum_groups_swap(h);
      if (rv[mb] && lg == 0) a.head_out[(int64_t)rb[mb] * N + rn[mb]] = live[mb] ? h + hb : 0.f;
      continue;
    }
    if (rv[mb]) {
      unsigned short* op = static_cast<unsigned short*>(a.out) + (int64_t)rb[mb] * a.o_sb +
                           (int64_t)rn[mb] * a.o_sn + lg * 4;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = live[mb] ? v[nb][j] : 0.f;
        if constexpr (RESID) {
          const u32x2 rw = rcur[nb];
          const f32x4 g = P_g(nb);
          o[0] = fmaxf(bf16_lo(rw.x) + g[0] * o[0], 0.f);
          o[1] = fmaxf(bf16_hi(rw.x) + g[1] * o[1], 0.f);
          o[2] = fmaxf(bf16_lo(rw.y) + g[2] * o[2], 0.f);
          o[3] = fmaxf(bf16_hi(rw.y) + g[3] * o[3], 0.f);
        }
        u32x2 pk;
        pk.x = pack_bf16x2(o[0], o[1]);
        pk.y = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<u32x2*>(op + nb * 16) = pk;
      }
    }
    if constexpr (RESID) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) rcur[nb] = rnext[nb];
    }
  }
}

// Global-gather variant: any N, any cin_pad; rows fetched from HBM / L2 per tap.
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
  conv_epilogue<COUT, MB, EPI, PS_GLOBAL>(a, acc, rb, rn, rv, lg);
}

// LDS-staged variant: one workgroup per position. The position's N rows
// (cin_pad = CIN channels) are copied once into LDS, plus one zero row at
// index N that stands for every absent neighbour, and all taps gather from
// there, so HBM sees each row once (the global variant re-fetches a row per
// tap once the rows of all resident positions exceed the L2).
// Row j occupies bytes [j*2*CIN, (j+1)*2*CIN); its 16-byte chunk c is stored
// at chunk slot c ^ (j % (CIN/8)), so the 16 lanes of an MFMA lane group,
// reading the same chunk of 16 different rows, mostly hit distinct banks.
template <int COUT, int MB, int EPI, int CIN>
__global__ __launch_bounds__(256, 2) void hex_conv_lds_kernel(const shrimp_conv_args a,
                                                              uint32_t w_bytes) {
  constexpr int NB = COUT / 16;
  constexpr int ROWB = CIN * 2;
  constexpr int CPR = CIN / 8;
  constexpr int KC = CIN / 32;
  constexpr int TILE = 4 * MB * 16;
  static_assert((CPR & (CPR - 1)) == 0, "chunks per row must be a power of two");
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int N = a.N;
  const int b = blockIdx.x;

  // ---- stage rows 0..N-1 and the zero row N --------------------------------
  {
    const unsigned short* xb = static_cast<const unsigned short*>(a.x) + (int64_t)b * a.x_sb;
    const int total = (N + 1) * CPR;
    constexpr int U = 8;
    for (int c0 = threadIdx.x; c0 < total; c0 += 256 * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 256;
        const int row = c / CPR;
        const int ch = c & (CPR - 1);
        v[u] = u32x4{0u, 0u, 0u, 0u};
        if (row < N) v[u] = *reinterpret_cast<const u32x4*>(xb + (int64_t)row * a.x_sn + ch * 8);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 256;
        const int row = c / CPR;
        const int ch = c & (CPR - 1);
        if (c < total)
          *reinterpret_cast<u32x4*>(xs + row * ROWB + ((ch ^ (row & (CPR - 1))) << 4)) = v[u];
      }
    }
  }
  __syncthreads();

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);
  const int* idxb = a.idx + (int64_t)b * N * a.idx_stride;
  const int taps = a.taps;
  const int nsteps = taps * KC;

  for (int tile0 = 0; tile0 < N; tile0 += TILE) {
    const int row_base = tile0 + wave * MB * 16;
    if (row_base >= N) break;
    int rb[MB], rn[MB];
    bool rv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      rb[mb] = b;
      rn[mb] = row_base + mb * 16 + lr;
      rv[mb] = rn[mb] < N;
    }
    // Neighbour row of tap t (N for absent) -> swizzled LDS row address.
    auto tap_rows = [&](int t, int (&j)[MB]) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        int v = rv[mb] ? idxb[rn[mb] * a.idx_stride + t] : N;
        j[mb] = (v >= 0 && v < N) ? v : N;
      }
    };
    auto row_addr = [&](int j) -> uint32_t {
      return (uint32_t)(j * ROWB) | ((uint32_t)(j & (CPR - 1)) << 4);
    };

    f32x4 acc[NB][MB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

    int jn[MB];
    uint32_t sw[MB];
    tap_rows(0, jn);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) sw[mb] = row_addr(jn[mb]);
    if (taps > 1) tap_rows(1, jn);

    u32x4 xf[MB], wf[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      xf[mb] = *reinterpret_cast<const u32x4*>(xs + (sw[mb] ^ ((uint32_t)lg << 4)));
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
        if (++kc == KC) {
          kc = 0;
          ++t;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) sw[mb] = row_addr(jn[mb]);
          if (t + 1 < taps) tap_rows(t + 1, jn);
        }
        const uint32_t cs = (uint32_t)(kc * 4 + lg) << 4;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          xf[mb] = *reinterpret_cast<const u32x4*>(xs + (sw[mb] ^ cs));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          wf[nb] = buf_load16(wr, (uint32_t)((((s + 1) * NB + nb) * 64 + lane) * 16));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma16x16x32(wc[nb], xc[mb], acc[nb][mb]);
    }
    conv_epilogue<COUT, MB, EPI, PS_GLOBAL>(a, acc, rb, rn, rv, lg);
  }
}

// Big-tile variant for the trunk shape (cin_pad = cout = 128, 7 taps, N <= 512):
// one workgroup per position with ceil(N/128) waves, each wave owning 128 rows
// x all 128 output channels (8 x 8 MFMA tiles, 256 fp32 accumulators held in
// AGPRs, so one wave per SIMD). Every weight fragment feeds 8 MFMAs and every
// gathered row fragment 8, which keeps both the L1 (weights) and the LDS (rows)
// well under their bandwidth at full MFMA rate.
//
// Rows are staged by buffer-to-LDS DMA (no registers, no LDS store
// instructions), channel-chunk-major: chunk kc (32 channels, 64 bytes) of row r
// sits at kc * NR * 64 + r * 64, its four 16-byte pieces swizzled as slot
// s = piece ^ ((r >> 2) & 3), so the 16 lanes of an MFMA lane group reading
// one piece of 16 different rows hit distinct banks. One DMA instruction
// fills 16 rows of one chunk; rows >= N (the zero row N for absent neighbours
// and the padding up to NR = ceil((N+1)/16)*16) read past the buffer and land
// as zeros. The K loop runs chunk-major (kc, then the 7 taps); chunk kc+1 is
// requested while chunk kc's MFMAs run, always after the step's weight
// prefetch (vmcnt retires in issue order, so a weight wait never waits for
// an HBM row load), and a barrier publishes it at the chunk boundary.
constexpr int BIG_MAX_N = 512;

SHRIMP_DEV int big_rows_padded(int N) { return ((N + 1 + 15) / 16) * 16; }

typedef __attribute__((address_space(3))) void lds_void_t;

template <int EPI>
__global__ __launch_bounds__(256, 1) void hex_conv_big_kernel(const shrimp_conv_args a,
                                                              uint32_t x_bytes, uint32_t w_bytes) {
  constexpr int COUT = 128, CIN = 128, KC = CIN / 32;
  constexpr int T = 7, MB = 8, NB = COUT / 16;
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int N = a.N;
  const int NR = big_rows_padded(N);
  const int groups = NR / 16;  // DMA instructions per chunk
  const int b = blockIdx.x;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const uint32_t xbase = (uint32_t)((int64_t)b * a.x_sb * 2);

  // DMA of chunk kc, rows [16 g, 16 g + 16): lane -> row 16 g + lane / 4, slot lane % 4.
  auto dma = [&](int kc, int g) {
    const int r = g * 16 + (lane >> 2);
    const int piece = (lane & 3) ^ ((r >> 2) & 3);
    const uint32_t off = r < N ? xbase + (uint32_t)(r * a.x_sn * 2) + (uint32_t)((kc * 4 + piece) * 16)
                               : SHRIMP_OOB_OFFSET;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        xr, (lds_void_t*)(xs + (kc * NR + g * 16) * 64), 16, off, 0, 0, 0);
  };

  // Prologue: chunk 0 by DMA, the neighbour indices of all taps, the first
  // weight fragments and the epilogue parameters, then one barrier.
  for (int g = wave; g < groups; g += nw) dma(0, g);
  const int row0 = wave * (MB * 16);
  int rn[MB], rb[MB];
  bool rv[MB];
  const int* idxb = a.idx + (int64_t)b * N * a.idx_stride;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    rb[mb] = b;
    rn[mb] = row0 + mb * 16 + lr;
    rv[mb] = rn[mb] < N;
  }
  int jr[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) jr[t][mb] = rv[mb] ? idxb[rn[mb] * a.idx_stride + t] : N;

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);
  auto wload = [&](int s, u32x4 (&w)[NB]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) w[nb] = buf_load16(wr, (uint32_t)(((s * NB + nb) * 64 + lane) * 16));
  };
  u32x4 wf[NB];
  wload(0, wf);

  // epilogue parameters after the rows: [bias | ln_w | ln_b | gamma or head_w]
  float* lp = reinterpret_cast<float*>(xs + KC * NR * 64);
  {
    const float* src[4] = {a.bias, a.ln_w, a.ln_b, (EPI & EPI_HEAD) ? a.head_w : a.gamma};
    for (int i = threadIdx.x; i < 4 * COUT; i += blockDim.x) {
      const float* sp = src[i / COUT];
      lp[i] = sp ? sp[i % COUT] : 0.f;
    }
  }

  // Neighbour rows as 16-bit row addresses within a chunk region:
  // j * 64 | ((j >> 2) & 3) << 4 (the piece swizzle); two per register.
  uint32_t sw2[T][MB / 2];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int m2 = 0; m2 < MB / 2; ++m2) {
      uint32_t pk = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = jr[t][2 * m2 + h];
        const int jj = (j >= 0 && j < N) ? j : N;
        pk |= (uint32_t)(jj * 64 + (((jj >> 2) & 3) << 4)) << (16 * h);
      }
      sw2[t][m2] = pk;
    }

  auto xload = [&](int t, int kc, u32x4 (&x)[MB]) {
    const uint32_t kbase = (uint32_t)(kc * NR * 64);
    const uint32_t ls = (uint32_t)lg << 4;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t v = (sw2[t][mb >> 1] >> (16 * (mb & 1))) & 0xFFFFu;
      x[mb] = *reinterpret_cast<const u32x4*>(xs + kbase + (v ^ ls));
    }
  };

  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Every wave owns rows (waves = ceil(N / 128)), so no wave skips the MFMAs;
  // the chunk loop is fully unrolled so that no value crosses a branch.
  const int mine = (groups - wave + nw - 1) / nw;  // DMA groups of this wave per chunk
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const bool more = kc + 1 < KC;
    u32x4 xf[MB];
    xload(0, kc, xf);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      u32x4 xc[MB], wc[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) xc[mb] = xf[mb];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wc[nb] = wf[nb];
      if (t + 1 < T) {
        xload(t + 1, kc, xf);
        wload((t + 1) * KC + kc, wf);
      } else if (more) {
        wload(kc + 1, wf);
      }
      if (more) {
        // this wave's DMA groups i in [i0, i1) of chunk kc + 1
        const int i0 = (t * mine) / T, i1 = ((t + 1) * mine) / T;
        for (int i = i0; i < i1; ++i) dma(kc + 1, wave + i * nw);
      }
      // Keep the next step's loads ahead of this step's MFMAs (the scheduler
      // would otherwise sink them next to their uses).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = mfma16x16x32(wc[nb], xc[mb], acc[nb][mb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of chunk kc + 1 has landed
      __syncthreads();
    }
  }
  conv_epilogue<COUT, MB, EPI, PS_LDS>(a, acc, rb, rn, rv, lg, lp);
}

// ---- weight packing ------------------------------------------------------------
// Fragment f = (ks * NB + nb) * 64 + lane holds 8 bf16, element e:
//   W[k][n = 16*nb + lane%16] with
//   k = 32*ks + 8*(lane/16) + e                    (standard order), or
//   k = 32*ks + 16*(e/4) + 4*(lane/16) + e%4       (interleaved order, used by
//       the fused MLP: the K-slice a lane holds is the 4 + 4 channels it owns
//       in the output fragments of the previous 16x16 MFMA product),
// and for convolutions k = t*cin_pad + c.
__global__ void pack_weight_kernel(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                   int K, int NOUT, int cin, int cin_pad, int64_t s_t,
                                   int64_t s_c, int64_t s_n, int interleaved) {
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
    const int k = interleaved ? ks * 32 + (e >> 2) * 16 + (lane >> 4) * 4 + (e & 3)
                              : ks * 32 + (lane >> 4) * 8 + e;
    const int t = k / cin_pad;
    const int c = k - t * cin_pad;
    const float v = (c < cin) ? src[t * s_t + c * s_c + n * s_n] : 0.f;
    dst[f * 8 + e] = f32_to_bf16_bits(v);
  }
}

template <int COUT, int MB, int EPI>
static int launch_conv(const shrimp_conv_args* a, uint32_t xb, uint32_t wb, size_t lds,
                       hipStream_t st) {
  if (COUT == 128 && lds && a->cin_pad == 128 && a->taps == 7 && a->N <= BIG_MAX_N &&
      (g_conv_variant == 0 || g_conv_variant == 3)) {
    const int waves = (a->N + 127) / 128;
    const int nr = ((a->N + 1 + 15) / 16) * 16;
    const size_t big_lds = (size_t)nr * 256 + 4 * 128 * sizeof(float);
    if (big_lds <= (size_t)max_lds_per_block()) {
      hipLaunchKernelGGL((hex_conv_big_kernel<EPI>), dim3(a->B), dim3(64 * waves), big_lds, st, *a,
                         xb, wb);
      return check_launch("hex_conv");
    }
    return check_launch("hex_conv");
  }
  if (lds) {
    switch (a->cin_pad) {
#define SHRIMP_CONV_LDS(CINV)                                                               \
  case CINV:                                                                                \
    hipLaunchKernelGGL((hex_conv_lds_kernel<COUT, MB, EPI, CINV>), dim3(a->B), dim3(256), lds, \
                       st, *a, wb);                                                         \
    return check_launch("hex_conv");
      SHRIMP_CONV_LDS(32)
      SHRIMP_CONV_LDS(64)
      SHRIMP_CONV_LDS(128)
#undef SHRIMP_CONV_LDS
      default:
        break;
    }
  }
  const int rows = a->B * a->N;
  const int per_block = 4 * MB * 16;
  const int grid = (rows + per_block - 1) / per_block;
  hipLaunchKernelGGL((hex_conv_kernel<COUT, MB, EPI>), dim3(grid), dim3(256), 0, st, *a, xb, wb);
  return check_launch("hex_conv");
}

template <int EPI>
static int dispatch_cout(const shrimp_conv_args* a, uint32_t xb, uint32_t wb, size_t lds,
                         hipStream_t st) {
  switch (a->cout) {
    case 32: return launch_conv<32, 4, EPI>(a, xb, wb, lds, st);
    case 64: return launch_conv<64, 4, EPI>(a, xb, wb, lds, st);
    case 96: return launch_conv<96, 4, EPI>(a, xb, wb, lds, st);
    case 128: return launch_conv<128, 4, EPI>(a, xb, wb, lds, st);
    case 192: return launch_conv<192, 2, EPI>(a, xb, wb, lds, st);
    case 256: return launch_conv<256, 1, EPI>(a, xb, wb, lds, st);
    default: return set_error(SHRIMP_EINVAL, "hex_conv: unsupported cout %d", a->cout);
  }
}

// LDS bytes the staged variant needs, or 0 when the global-gather variant
// runs instead (cin_pad without a staged instance, unaligned rows, or a
// position too large for one workgroup's LDS).
static size_t conv_lds_bytes(const shrimp_conv_args* a) {
  if (a->cin_pad != 32 && a->cin_pad != 64 && a->cin_pad != 128) return 0;
  if ((reinterpret_cast<uintptr_t>(a->x) & 15) != 0 || a->x_sb % 8 != 0 || a->x_sn % 8 != 0)
    return 0;
  const size_t bytes = (size_t)(a->N + 1) * a->cin_pad * 2;
  return bytes <= (size_t)max_lds_per_block() ? bytes : 0;
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
                     (int64_t)cin * cout, (int64_t)cout, (int64_t)1, 0);
  return check_launch("pack_conv_weight");
}

static int pack_linear(const float* w, void* packed, int in_features, int out_features,
                       void* stream, int interleaved) {
  SHRIMP_REQUIRE(w && packed, "pack_linear_weight: null pointer");
  SHRIMP_REQUIRE(in_features % 32 == 0 && out_features % 16 == 0,
                 "pack_linear_weight: shape (%d -> %d) needs in %% 32 == 0, out %% 16 == 0",
                 in_features, out_features);
  const int64_t frags = (int64_t)(in_features / 32) * (out_features / 16) * 64;
  const int grid = (int)((frags + 255) / 256);
  hipLaunchKernelGGL(pack_weight_kernel, dim3(grid), dim3(256), 0, as_stream(stream), w,
                     static_cast<unsigned short*>(packed), in_features, out_features,
                     in_features, in_features, (int64_t)0, (int64_t)1, (int64_t)in_features,
                     interleaved);
  return check_launch("pack_linear_weight");
}

extern "C" int shrimp_pack_linear_weight(const float* w, void* packed, int in_features,
                                         int out_features, void* stream) {
  return pack_linear(w, packed, in_features, out_features, stream, 0);
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
  const size_t lds = g_conv_variant == 1 ? 0 : conv_lds_bytes(a);
  if (head) {
    SHRIMP_REQUIRE(a->relu, "hex_conv: head epilogue expects relu");
    return dispatch_cout<EPI_HEAD | EPI_RELU>(a, xb, wb, lds, st);
  }
  if (resid) {
    SHRIMP_REQUIRE(ln && !a->relu, "hex_conv: residual epilogue is LN (no relu) + residual");
    return dispatch_cout<EPI_LN | EPI_RESID>(a, xb, wb, lds, st);
  }
  if (ln) {
    return a->relu ? dispatch_cout<EPI_LN | EPI_RELU>(a, xb, wb, lds, st)
                   : dispatch_cout<EPI_LN>(a, xb, wb, lds, st);
  }
  return a->relu ? dispatch_cout<EPI_RELU>(a, xb, wb, lds, st)
                 : dispatch_cout<0>(a, xb, wb, lds, st);
}
