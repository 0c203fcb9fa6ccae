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
#include <type_traits>

#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

// EPI_BACC: the accumulators started from the bias (no bias add here).
enum : int { EPI_LN = 1, EPI_RELU = 2, EPI_RESID = 4, EPI_HEAD = 8, EPI_BACC = 16 };

// ReLU of two packed bf16: as 16-bit integers, every value with the sign bit
// set is below 0, so a packed integer max against 0 is the float max.
SHRIMP_DEV unsigned relu_bf16x2(unsigned w) {
  typedef __attribute__((ext_vector_type(2))) short s16x2;
  const s16x2 v = __builtin_bit_cast(s16x2, w);
  return __builtin_bit_cast(unsigned, __builtin_elementwise_max(v, s16x2{0, 0}));
}

// Bias / LayerNorm / ReLU / mask / residual / head epilogue on the fp32
// accumulators of MB row blocks. rb, rn: position and cell index of this
// lane's row in block mb; rv: row exists.
// Per-channel parameters (PSRC): PS_GLOBAL reads them where used; PS_REGS
// loads this lane's channels once into registers (re-reading after a store
// would wait, since the compiler must assume the store may alias them);
// PS_LDS reads them from an LDS copy at `lp` laid out [bias | ln_w | ln_b |
// gamma or head_w | zeros], COUT floats each. With LDS parameters a masked
// row gets LayerNorm scale 0 and its ln_b from the zero slot, so the
// LayerNorm itself yields exact zeros and no per-value select is needed.
// The residual rows are requested RD blocks ahead of their use.
// `store(mb, nb, u32x2)` receives 4 packed bf16 channels 16 nb + 4 lg .. + 3
// of row block mb, for rows that exist.
enum : int { PS_GLOBAL = 0, PS_REGS = 1, PS_LDS = 2, PS_LDSREG = 3 };

// Store functors with a `kBuffered` member write through a buffer resource and
// take every row, absent ones at an offset past the resource (dropped); with
// them the epilogue also reads the residual rows through the functor's
// `rres` resource, absent rows reading zeros. No load or store then sits under
// a per-row branch, so waiting for a prefetched residual row counts exactly
// the requests issued after it (memory operations retire in order; a branch
// makes the compiler assume the fewest and wait for every earlier store).
template <class T, class = void>
struct is_buffered_store : std::false_type {};
template <class T>
struct is_buffered_store<T, std::void_t<decltype(T::kBuffered)>> : std::true_type {};

template <int COUT, int MB, int EPI, int PSRC, typename Store>
SHRIMP_DEV void conv_epilogue(const shrimp_conv_args& a, f32x4 (&acc)[COUT / 16][MB],
                              const int (&rb)[MB], const int (&rn)[MB], const bool (&rv)[MB],
                              int lg, const float* lp, Store&& store) {
  constexpr int NB = COUT / 16;
  constexpr bool LN = (EPI & EPI_LN) != 0, RESID = (EPI & EPI_RESID) != 0;
  constexpr bool HEAD = (EPI & EPI_HEAD) != 0, RELU = (EPI & EPI_RELU) != 0;
  constexpr bool BACC = (EPI & EPI_BACC) != 0;
  constexpr bool PRE = PSRC == PS_REGS;
  constexpr bool BUF = is_buffered_store<std::remove_cv_t<std::remove_reference_t<Store>>>::value;
  constexpr bool FROM_LDS = PSRC == PS_LDS || PSRC == PS_LDSREG;
  constexpr bool HREG = PSRC == PS_LDSREG;  // bias / ln_w read from LDS once, kept in registers
  constexpr bool LNMASK = LN && FROM_LDS;   // masking folded into the LayerNorm
  constexpr int PN = PRE ? NB : 1;
  constexpr int RD = MB < 3 ? MB : 3;  // residual prefetch depth (row blocks)
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
    if constexpr (FROM_LDS) return prm(lp + slot * COUT, nb);
    else if constexpr (PRE) return r[ri];
    else return prm(g, nb);
  };
  f32x4 hb_[HREG ? NB : 1], hw_[HREG ? NB : 1];
  if constexpr (HREG) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      hb_[nb] = prm(lp, nb);
      hw_[nb] = prm(lp + COUT, nb);
    }
  }
  auto P_b = [&](int nb) {
    if constexpr (HREG) return hb_[nb];
    else return pick(0, a.bias, pb, nb, nb);
  };
  auto P_w = [&](int nb) {
    if constexpr (HREG) return hw_[nb];
    else return pick(1, a.ln_w, pw, nb, LN && PRE ? nb : 0);
  };
  auto P_l = [&](int nb) { return pick(2, a.ln_b, pl, nb, LN && PRE ? nb : 0); };
  auto P_g = [&](int nb) { return pick(3, a.gamma, pg, nb, RESID && PRE ? nb : 0); };
  auto P_h = [&](int nb) { return pick(3, a.head_w, ph, nb, HEAD && PRE ? nb : 0); };
  bool live[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) live[mb] = rv[mb] && a.mask[(int64_t)rb[mb] * N + rn[mb]] != 0;
  const float hb = HEAD ? a.head_b[0] : 0.f;

  auto resid_row = [&](int mb, u32x2 (&r)[NB]) {
    if constexpr (RESID && BUF) {
      const uint32_t ro =
          rv[mb] ? (uint32_t)(((int64_t)rb[mb] * a.r_sb + (int64_t)rn[mb] * a.r_sn + lg * 4) * 2)
                 : SHRIMP_OOB_OFFSET;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) r[nb] = buf_load8(store.rres, ro + nb * 32);
    } else if constexpr (RESID) {
      const unsigned short* rp = static_cast<const unsigned short*>(a.resid) +
                                 (int64_t)rb[mb] * a.r_sb + (int64_t)rn[mb] * a.r_sn + lg * 4;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        r[nb] = rv[mb] ? *reinterpret_cast<const u32x2*>(rp + nb * 16) : u32x2{0u, 0u};
    }
  };
  u32x2 rbuf[RESID ? RD : 1][RESID ? NB : 1];
  if constexpr (RESID) {
#pragma unroll
    for (int i = 0; i < RD; ++i) resid_row(i, rbuf[i]);
  }

#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float v[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (BACC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[nb][j] = acc[nb][mb][j];
      } else {
        const f32x4 bb = P_b(nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[nb][j] = acc[nb][mb][j] + bb[j];
      }
    }
    if constexpr (LN) {
      // one pass for the row statistics: sum and sum of squares in four
      // independent chains (one per element j), variance = E[v^2] - mean^2
      // (the pre-LN conv outputs have |mean| of the order of their spread, so
      // fp32 keeps the difference to about 2^-22 relative); each value then
      // takes two FMAs: (v * rstd - mean * rstd) * ln_w + ln_b
      float sj[4], qj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sj[j] = v[0][j];
        qj[j] = v[0][j] * v[0][j];
#pragma unroll
        for (int nb = 1; nb < NB; ++nb) {
          sj[j] += v[nb][j];
          qj[j] = fmaf(v[nb][j], v[nb][j], qj[j]);
        }
      }
      const float mean = sum_groups_swap((sj[0] + sj[1]) + (sj[2] + sj[3])) * (1.0f / COUT);
      const float ex2 = sum_groups_swap((qj[0] + qj[1]) + (qj[2] + qj[3])) * (1.0f / COUT);
      float rstd = rsqrtf(fmaxf(fmaf(-mean, mean, ex2), 0.f) + a.eps);
      int bslot = 2;
      if constexpr (LNMASK) {
        rstd = live[mb] ? rstd : 0.f;
        bslot = live[mb] ? 2 : 4;
      }
      const float nmr = -mean * rstd;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 gw = P_w(nb);
        const f32x4 gb = LNMASK ? prm(lp + bslot * COUT, nb) : P_l(nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[nb][j] = fmaf(fmaf(v[nb][j], rstd, nmr), gw[j], gb[j]);
      }
    }
    if constexpr (HEAD) {
      if constexpr (RELU) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j) v[nb][j] = relu_bits(v[nb][j]);
      }
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
    // ReLU and the row mask in one clamp: med3(v, 0, +inf) = relu(v), med3(v, 0, 0) = 0.
    const float cap = live[mb] ? __builtin_inff() : 0.f;
    if (BUF || rv[mb]) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (LNMASK) o[j] = v[nb][j];
          else if constexpr (RELU && !RESID) o[j] = __builtin_amdgcn_fmed3f(v[nb][j], 0.f, cap);
          else o[j] = live[mb] ? v[nb][j] : 0.f;
        }
        if constexpr (RESID) {
          const u32x2 rw = rbuf[mb % RD][nb];
          const f32x4 g = P_g(nb);
          o[0] = fmaf(g[0], o[0], bf16_lo(rw.x));
          o[1] = fmaf(g[1], o[1], bf16_hi(rw.x));
          o[2] = fmaf(g[2], o[2], bf16_lo(rw.y));
          o[3] = fmaf(g[3], o[3], bf16_hi(rw.y));
        }
        u32x2 pk;
        pk.x = pack_bf16x2(o[0], o[1]);
        pk.y = pack_bf16x2(o[2], o[3]);
        // the residual block's ReLU, and ReLU after a masking LayerNorm, on the
        // rounded values (the same result as before rounding)
        if constexpr (RESID || (LNMASK && RELU)) {
          pk.x = relu_bf16x2(pk.x);
          pk.y = relu_bf16x2(pk.y);
        }
        store(mb, nb, pk);
      }
    }
    if constexpr (RESID) {
      if (mb + RD < MB) resid_row(mb + RD, rbuf[mb % RD]);
    }
  }
}

// Store functor of the epilogue: rows of `a.out` (bf16, strides o_sb / o_sn).
template <int MB>
struct GlobalRowStore {
  unsigned short* p[MB];
  SHRIMP_DEV GlobalRowStore(const shrimp_conv_args& a, const int (&rb)[MB], const int (&rn)[MB],
                            int lg) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      p[mb] = static_cast<unsigned short*>(a.out) + (int64_t)rb[mb] * a.o_sb +
              (int64_t)rn[mb] * a.o_sn + lg * 4;
  }
  SHRIMP_DEV void operator()(int mb, int nb, u32x2 pk) const {
    *reinterpret_cast<u32x2*>(p[mb] + nb * 16) = pk;
  }
};

// Store functor for 128-channel rows with 16-byte stores: the output blocks
// come in pairs (nb even, then nb + 1); one lane-group swap (v_permlane16_swap)
// gives each lane 8 adjacent channels, lane group g of the pair's 32 channels
// taking 8 g' .. 8 g' + 7 with g' = 2 (g & 1) + (g >> 1), so the four lane
// groups of a row cover its 64 bytes. Needs o_sb, o_sn multiples of 8 and a
// 16-byte aligned output; rows of a lane group exist or not together.
template <int MB>
struct GlobalRowStore16 {
  unsigned short* p[MB];
  u32x2 pend;
  SHRIMP_DEV GlobalRowStore16(const shrimp_conv_args& a, const int (&rb)[MB], const int (&rn)[MB],
                              int lg) {
    const int sub = (lg & 1) * 16 + (lg >> 1) * 8;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      p[mb] = static_cast<unsigned short*>(a.out) + (int64_t)rb[mb] * a.o_sb +
              (int64_t)rn[mb] * a.o_sn + sub;
  }
  SHRIMP_DEV void operator()(int mb, int nb, u32x2 pk) {
    if ((nb & 1) == 0) {
      pend = pk;
      return;
    }
    // even rows of a 16-lane pair keep their block-nb channels and receive the
    // partner's; odd rows receive the partner's block-(nb+1) channels
    const auto sx = __builtin_amdgcn_permlane16_swap(pend.x, pk.x, false, false);
    const auto sy = __builtin_amdgcn_permlane16_swap(pend.y, pk.y, false, false);
    *reinterpret_cast<u32x4*>(p[mb] + (nb >> 1) * 32) = u32x4{sx[0], sy[0], sx[1], sy[1]};
  }
};

// GlobalRowStore16 through buffer resources (see is_buffered_store): `out`
// spans o_bytes, the residual rows `rres` r_bytes.
// A row block's byte offset is computed at its first store (nb = 0), so only
// the current block's offset is held in a register through the epilogue.
template <int MB>
struct BufRowStore16 {
  static constexpr bool kBuffered = true;
  __amdgpu_buffer_rsrc_t orr, rres;
  const int (&rb)[MB];
  const int (&rn)[MB];
  const bool (&rv)[MB];
  int64_t o_sb, o_sn;
  int sub;
  uint32_t cur = 0;
  u32x2 pend;
  SHRIMP_DEV BufRowStore16(const shrimp_conv_args& a, const int (&rb_)[MB], const int (&rn_)[MB],
                           const bool (&rv_)[MB], int lg, uint32_t o_bytes, uint32_t r_bytes)
      : orr(make_rsrc(a.out, o_bytes)), rres(make_rsrc(a.resid, r_bytes)), rb(rb_), rn(rn_),
        rv(rv_), o_sb(a.o_sb), o_sn(a.o_sn), sub((lg & 1) * 16 + (lg >> 1) * 8) {}
  SHRIMP_DEV void operator()(int mb, int nb, u32x2 pk) {
    if ((nb & 1) == 0) {
      if (nb == 0)
        cur = rv[mb] ? (uint32_t)(((int64_t)rb[mb] * o_sb + (int64_t)rn[mb] * o_sn + sub) * 2)
                     : SHRIMP_OOB_OFFSET;
      pend = pk;
      return;
    }
    const auto sx = __builtin_amdgcn_permlane16_swap(pend.x, pk.x, false, false);
    const auto sy = __builtin_amdgcn_permlane16_swap(pend.y, pk.y, false, false);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{sx[0], sy[0], sx[1], sy[1]}, orr,
                                           cur + (uint32_t)((nb >> 1) * 64), 0, 0);
  }
};

template <int COUT, int MB, int EPI, int PSRC>
SHRIMP_DEV void conv_epilogue(const shrimp_conv_args& a, f32x4 (&acc)[COUT / 16][MB],
                              const int (&rb)[MB], const int (&rn)[MB], const bool (&rv)[MB],
                              int lg, const float* lp = nullptr) {
  if constexpr ((EPI & EPI_HEAD) != 0) {
    conv_epilogue<COUT, MB, EPI, PSRC>(a, acc, rb, rn, rv, lg, lp, [](int, int, u32x2) {});
  } else {
    conv_epilogue<COUT, MB, EPI, PSRC>(a, acc, rb, rn, rv, lg, lp, GlobalRowStore<MB>(a, rb, rn, lg));
  }
}

// Global-gather variant: any N, any cin_pad; rows fetched from HBM / L2 per tap.
template <int COUT, int MB, int EPI>
__global__ __launch_bounds__(256, 2) void hex_conv_kernel(const shrimp_conv_args a,
                                                          uint32_t x_bytes, uint32_t w_bytes) {
  constexpr int NB = COUT / 16;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
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
      SHRIMP_DCHECK(j >= -1, SHRIMP_DBG_CONV_INDEX);
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

// Per-channel parameters of an LDS-parameter epilogue (PS_LDS): [bias | ln_w |
// ln_b | gamma or head_w | zeros], COUT floats each, absent ones zero.
template <int COUT>
SHRIMP_DEV void stage_params(float* lp, const shrimp_conv_args& a, bool head) {
  const float* extra = head ? a.head_w : a.gamma;
  for (int i = threadIdx.x; i < 5 * COUT; i += blockDim.x) {
    const int slot = i / COUT, c = i - slot * COUT;
    const float* sp = slot == 0 ? a.bias : slot == 1 ? a.ln_w : slot == 2 ? a.ln_b : slot == 3 ? extra : nullptr;
    lp[i] = sp ? sp[c] : 0.f;
  }
}

// Epilogue of the LDS-staged conv: parameters from LDS; B16: 16-byte stores
// (and residual reads) through buffer resources over o_bytes / r_bytes.
template <int COUT, int MB, int EPI, bool B16>
SHRIMP_DEV void lds_conv_epilogue(const shrimp_conv_args& a, f32x4 (&acc)[COUT / 16][MB],
                                  const int (&rb)[MB], const int (&rn)[MB], const bool (&rv)[MB],
                                  int lg, const float* lp, uint32_t o_bytes, uint32_t r_bytes) {
  if constexpr ((EPI & EPI_HEAD) != 0) {
    conv_epilogue<COUT, MB, EPI, PS_LDS>(a, acc, rb, rn, rv, lg, lp, [](int, int, u32x2) {});
  } else if constexpr (B16) {
    conv_epilogue<COUT, MB, EPI, PS_LDS>(a, acc, rb, rn, rv, lg, lp,
                                         BufRowStore16<MB>(a, rb, rn, rv, lg, o_bytes, r_bytes));
  } else {
    conv_epilogue<COUT, MB, EPI, PS_LDS>(a, acc, rb, rn, rv, lg, lp, GlobalRowStore<MB>(a, rb, rn, lg));
  }
}

// LDS-staged variant: workgroups (position, row split); split y of Y takes the
// row tiles y, y + Y, ... (Y = 1 for batches that fill the GPU; small batches
// spread a position's tiles over several workgroups, each staging all rows). The position's N rows
// (cin_pad = CIN channels) are copied once into LDS, plus one zero row at
// index N that stands for every absent neighbour, and all taps gather from
// there, so HBM sees each row once (the global variant re-fetches a row per
// tap once the rows of all resident positions exceed the L2).
// Row j occupies bytes [j*2*CIN, (j+1)*2*CIN); its 16-byte chunk c is stored
// at chunk slot c ^ (j % (CIN/8)), so the 16 lanes of an MFMA lane group,
// reading the same chunk of 16 different rows, mostly hit distinct banks.
// BIGORDER (7 taps): the big-tile kernel's arithmetic, so a small batch split
// over workgroups gives the same bits as the large batch: accumulators start
// from the bias (except for the residual epilogue) and the K loop runs channel
// chunk outer, tap inner.
// The per-channel parameters follow the rows in LDS (stage_params); B16: see
// lds_conv_epilogue.
template <int COUT, int MB, int EPI, int CIN, bool BIGORDER = false, bool B16 = false>
__global__ __launch_bounds__(256, 2) void hex_conv_lds_kernel(const shrimp_conv_args a,
                                                              uint32_t w_bytes, uint32_t o_bytes,
                                                              uint32_t r_bytes) {
  constexpr int NB = COUT / 16;
  constexpr int ROWB = CIN * 2;
  constexpr int CPR = CIN / 8;
  constexpr int KC = CIN / 32;
  constexpr int TILE = 4 * MB * 16;
  static_assert((CPR & (CPR - 1)) == 0, "chunks per row must be a power of two");
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
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
  float* lp = reinterpret_cast<float*>(xs + (((N + 1) * ROWB + 15) & ~15));
  stage_params<COUT>(lp, a, (EPI & EPI_HEAD) != 0);
  __syncthreads();

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);
  const int* idxb = a.idx + (int64_t)b * N * a.idx_stride;
  const int taps = a.taps;
  const int nsteps = taps * KC;

  for (int tile0 = (int)blockIdx.y * TILE; tile0 < N; tile0 += (int)gridDim.y * TILE) {
    const int row_base = tile0 + wave * MB * 16;
    // BIGORDER waves meet at barriers in the K loop, so a wave without rows
    // runs it (on the zero row) and skips only the epilogue.
    if (!BIGORDER && row_base >= N) break;
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
        SHRIMP_DCHECK(v >= -1, SHRIMP_DBG_CONV_INDEX);
        j[mb] = (v >= 0 && v < N) ? v : N;
      }
    };
    auto row_addr = [&](int j) -> uint32_t {
      return (uint32_t)(j * ROWB) | ((uint32_t)(j & (CPR - 1)) << 4);
    };

    f32x4 acc[NB][MB];
    if constexpr (BIGORDER) {
      constexpr bool BA = (EPI & EPI_RESID) == 0;
      constexpr int T = 7;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 bb = BA ? *reinterpret_cast<const f32x4*>(a.bias + nb * 16 + lg * 4)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = bb;
      }
      uint32_t sa[T][MB];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        int j[MB];
        tap_rows(t, j);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sa[t][mb] = row_addr(j[mb]);
      }
      // A step's weight fragments (NB x 1 KiB, contiguous) are loaded once per
      // workgroup, 16 bytes per thread and piece, D steps ahead in registers,
      // and handed to the waves through one LDS buffer: each wave reads its
      // fragments, a barrier, the next step's pieces are stored, a barrier.
      // (Per wave, the same fragments in the same MFMA order as a per-wave
      // load, so the same bits; a quarter of the L2 reads, and a prefetch
      // deep enough for a step's 8 MFMAs to cover the L2 latency.) Row
      // fragments run one step ahead from the staged rows.
      constexpr int NS = T * KC;
      constexpr int WP = NB * 64;            // 16-byte pieces per step
      constexpr int WPT = (WP + 255) / 256;  // per thread
      constexpr int D = 6;                   // steps in flight
      __shared__ u32x4 wls[WP];
      u32x4 stg[D][WPT], wq[NB], xq[2][MB];
      auto gload = [&](int s, u32x4 (&r)[WPT]) {
        const int kc = s / T, t = s % T;
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
          const int i = (int)threadIdx.x + k * 256;
          if (WP % 256 == 0 || i < WP)
            r[k] = buf_load16(wr, (uint32_t)(((t * KC + kc) * WP + i) * 16));
        }
      };
      auto sstore = [&](const u32x4 (&r)[WPT]) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
          const int i = (int)threadIdx.x + k * 256;
          if (WP % 256 == 0 || i < WP) wls[i] = r[k];
        }
      };
      auto load_x = [&](int s, u32x4 (&x)[MB]) {
        const int kc = s / T, t = s % T;
        const uint32_t cs = (uint32_t)(kc * 4 + lg) << 4;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) x[mb] = *reinterpret_cast<const u32x4*>(xs + (sa[t][mb] ^ cs));
      };
#pragma unroll
      for (int d = 0; d < D && d < NS; ++d) gload(d, stg[d]);
      __syncthreads();  // the previous tile's last fragments are read
      sstore(stg[0]);
      if (D < NS) gload(D, stg[0]);
      load_x(0, xq[0]);
      __syncthreads();
#pragma unroll
      for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) wq[nb] = wls[nb * 64 + lane];
        if (s + 1 < NS) load_x(s + 1, xq[(s + 1) % 2]);
        if (s + 1 < NS) __syncthreads();  // every wave holds step s's fragments
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[nb][mb] = mfma16x16x32(wq[nb], xq[s % 2][mb], acc[nb][mb]);
        if (s + 1 < NS) {
          sstore(stg[(s + 1) % D]);
          if (s + 1 + D < NS) gload(s + 1 + D, stg[(s + 1) % D]);
          __syncthreads();  // step s + 1's fragments are visible
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (row_base >= N) continue;
      lds_conv_epilogue<COUT, MB, BA ? (EPI | EPI_BACC) : EPI, B16>(a, acc, rb, rn, rv, lg, lp,
                                                                   o_bytes, r_bytes);
      continue;
    }
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
    lds_conv_epilogue<COUT, MB, EPI, B16>(a, acc, rb, rn, rv, lg, lp, o_bytes, r_bytes);
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
// as zeros. All four chunks are requested before the K loop: staging them
// during the MFMA phases instead costs more than it hides, because vmcnt
// retires in issue order and every weight load issued after a row DMA waits
// for it. The K loop runs chunk-major (kc, then the 7 taps).
constexpr int BIG_MAX_N = 512;
// Two workgroups of three waves per position (hex_conv_big_kernel with
// gridDim.y = 2): up to 3 * 128 rows per half, and ceil((N + 1) / 16) <= 3 *
// BIG_SPLIT_GPW row groups staged by each.
constexpr int BIG_SPLIT_MAX_N = 576;
constexpr int BIG_SPLIT_GPW = 13;
constexpr int BIG_SPLIT_MIN_B = 32;
constexpr int BIG_PARAMS = 5 * 128;  // floats: [bias | ln_w | ln_b | gamma or head_w | zeros]

__host__ __device__ inline int big_rows_padded(int N) { return ((N + 1 + 15) / 16) * 16; }

typedef __attribute__((address_space(3))) void lds_void_t;

// Per-wave state of a big-tile workgroup (position b, rows 128 wave .. + 127).
struct BigTile {
  int lane, wave, nw, lg, N, NR, groups, b;
  __amdgpu_buffer_rsrc_t xr;
  uint32_t xbase, xsn2;
  int rb[8], rn[8];
  bool rv[8];
  uint32_t sw2[7][4];  // neighbour row addresses, two 16-bit values per register
};

// Row ids and validity of a whole-position workgroup's wave (rows 128 wave ..
// + 127 below N), recomputed from an opaque copy of the lane id before an
// epilogue, so they are not held in registers across the conv passes.
SHRIMP_DEV void big_rows(BigTile& t) {
  int lane = t.lane;
  asm volatile("" : "+v"(lane));
  const int row0 = t.wave * 128;
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    t.rn[mb] = row0 + mb * 16 + (lane & 15);
    t.rv[mb] = t.rn[mb] < t.N;
  }
}

// DMA of chunk kc, rows [16 g, 16 g + 16): lane -> row 16 g + lane / 4, slot lane % 4.
SHRIMP_DEV void big_dma(unsigned char* xs, const BigTile& t, int kc, int g) {
  const int r = g * 16 + (t.lane >> 2);
  const int piece = (t.lane & 3) ^ ((r >> 2) & 3);
  const uint32_t off = r < t.N ? t.xbase + (uint32_t)r * t.xsn2 + (uint32_t)((kc * 4 + piece) * 16)
                               : SHRIMP_OOB_OFFSET;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(t.xr, (lds_void_t*)(xs + (kc * t.NR + g * 16) * 64), 16,
                                           off, 0, 0, 0);
}

// Epilogue parameters of NS convs, [bias | ln_w | ln_b | extra | zeros] of
// 128 floats each in LDS. They are requested into registers before the row
// DMA (memory requests retire in order, so a wait for them issued after the
// DMA would wait for the rows as well) and written to LDS once it is issued.
// Slot s = tid + j * blockDim.x (j = 0, 1; stored when s < 128) carries
// floats 4 (s & 31) .. + 3 of array s >> 5; a null array stores zeros.
template <int NS>
struct BigParams {
  f32x4 v[NS][2];
  SHRIMP_DEV void load(int set, const float* bias, const float* ln_w, const float* ln_b,
                       const float* extra) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int sl = (int)(threadIdx.x + j * blockDim.x) & 127;
      const int arr = sl >> 5;
      const float* src = arr == 0 ? bias : (arr == 1 ? ln_w : (arr == 2 ? ln_b : extra));
      const float* p = src ? src : bias;
      const f32x4 x = *reinterpret_cast<const f32x4*>(p + 4 * (sl & 31));
      v[set][j] = src ? x : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  SHRIMP_DEV void store(float* lp) const {
#pragma unroll
    for (int set = 0; set < NS; ++set) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int sl = (int)(threadIdx.x + j * blockDim.x);
        if (sl < 128)
          *reinterpret_cast<f32x4*>(lp + set * BIG_PARAMS + (sl >> 5) * 128 + 4 * (sl & 31)) = v[set][j];
      }
      if (threadIdx.x < 32)
        *reinterpret_cast<f32x4*>(lp + set * BIG_PARAMS + 512 + 4 * threadIdx.x) =
            f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// Requests all four chunks by DMA and turns the neighbour indices of this wave's rows
// into swizzled 16-bit LDS row addresses j * 64 | ((j >> 2) & 3) << 4.
// The indices are requested before the rows (three loads per row block, absent
// rows reading zeros past the resource), and every wave issues the same GPW
// DMAs per chunk (a wave with fewer groups repeats its first one: the same
// bytes to the same place), so the wait for the indices counts the DMAs
// instead of waiting for them and the row addresses are computed while the
// rows arrive. Needs idx_stride >= 7 and ceil((N + 1) / 16) <= GPW * waves.
// The workgroup computes rows [rbase, rend) (128 per wave from rbase); every
// workgroup stages all rows of its position, since the taps reach anywhere in
// it.
template <int GPW = 9>
SHRIMP_DEV void big_setup(BigTile& t, const shrimp_conv_args& a, unsigned char* xs,
                          uint32_t x_bytes, int rbase = 0, int rend = 1 << 30) {
  // DMAs per chunk and wave: with ceil(N / 128) waves over the whole position
  // a wave owns at most ceil((8 nw + 1) / nw) = 9 of the ceil((N + 1) / 16)
  // row groups (GPW = 9)
  constexpr int T = 7, MB = 8;
  t.lane = threadIdx.x & 63;
  t.wave = wave_id();
  t.nw = blockDim.x >> 6;
  t.lg = t.lane >> 4;
  t.N = a.N;
  t.NR = big_rows_padded(a.N);
  t.groups = t.NR / 16;
  t.b = blockIdx.x;
  t.xr = make_rsrc(a.x, x_bytes);
  t.xbase = (uint32_t)((int64_t)t.b * a.x_sb * 2);
  t.xsn2 = (uint32_t)(a.x_sn * 2);
  const int row0 = rbase + t.wave * (MB * 16);
  const int rlim = rend < t.N ? rend : t.N;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    t.rb[mb] = t.b;
    t.rn[mb] = row0 + mb * 16 + (t.lane & 15);
    t.rv[mb] = t.rn[mb] < rlim;
  }
  const __amdgpu_buffer_rsrc_t ir =
      make_rsrc(a.idx + (int64_t)t.b * t.N * a.idx_stride, (uint32_t)(t.N * a.idx_stride * 4));
  u32x4 i0[MB];
  u32x2 i1[MB];
  unsigned i2[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const uint32_t off = t.rv[mb] ? (uint32_t)(t.rn[mb] * a.idx_stride * 4) : SHRIMP_OOB_OFFSET;
    i0[mb] = buf_load16(ir, off);
    i1[mb] = buf_load8(ir, off + 16);
    i2[mb] = buf_load4(ir, off + 24);
  }
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
      const int g = t.wave + i * t.nw;
      big_dma(xs, t, kc, g < t.groups ? g : t.wave);
    }
#pragma unroll
  for (int tp = 0; tp < T; ++tp)
#pragma unroll
    for (int m2 = 0; m2 < MB / 2; ++m2) {
      uint32_t pk = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int mb = 2 * m2 + h;
        const unsigned raw = tp < 4 ? i0[mb][tp] : (tp < 6 ? i1[mb][tp - 4] : i2[mb]);
        const int j = t.rv[mb] ? (int)raw : t.N;
        SHRIMP_DCHECK(j >= -1, SHRIMP_DBG_CONV_INDEX);
        const int jj = (j >= 0 && j < t.N) ? j : t.N;
        pk |= (uint32_t)(jj * 64 + (((jj >> 2) & 3) << 4)) << (16 * h);
      }
      t.sw2[tp][m2] = pk;
    }
}

// Weight fragments of k-step s (8 output blocks).
SHRIMP_DEV void big_wload(__amdgpu_buffer_rsrc_t wr, int s, int lane, u32x4 (&w)[8]) {
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) w[nb] = buf_load16(wr, (uint32_t)(((s * 8 + nb) * 64 + lane) * 16));
}

// Accumulators start from the conv bias (lane: channels 16 nb + 4 lg .. + 3).
SHRIMP_DEV void big_acc_init(f32x4 (&acc)[8][8], const float* bias, int lg) {
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const f32x4 bb = *reinterpret_cast<const f32x4*>(bias + nb * 16 + lg * 4);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc[nb][mb] = bb;
  }
}

// One 7-tap, 128 -> 128 conv over the rows in LDS: acc += sum_t W_t^T X[idx_t]^T.
// On entry wf holds k-step 0 of `wr`.
SHRIMP_DEV void big_pass(f32x4 (&acc)[8][8], u32x4 (&wf)[8], const BigTile& t,
                         unsigned char* xs, __amdgpu_buffer_rsrc_t wr) {
  constexpr int KC = 4, T = 7, MB = 8, NB = 8;
  auto xload = [&](int tp, int kc, u32x4 (&x)[MB]) {
    const uint32_t kbase = (uint32_t)(kc * t.NR * 64);
    const uint32_t ls = (uint32_t)t.lg << 4;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t v = (t.sw2[tp][mb >> 1] >> (16 * (mb & 1))) & 0xFFFFu;
      x[mb] = *reinterpret_cast<const u32x4*>(xs + kbase + (v ^ ls));
    }
  };
  // The chunk loop is fully unrolled so that no value crosses a branch. The
  // last tap of a chunk requests the next chunk's first rows and weights.
  u32x4 xf[MB];
  xload(0, 0, xf);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const bool more = kc + 1 < KC;
#pragma unroll
    for (int tp = 0; tp < T; ++tp) {
      u32x4 xc[MB], wc[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) xc[mb] = xf[mb];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wc[nb] = wf[nb];
      if (tp + 1 < T) {
        xload(tp + 1, kc, xf);
        big_wload(wr, (tp + 1) * KC + kc, t.lane, wf);
      } else if (more) {
        xload(0, kc + 1, xf);
        big_wload(wr, kc + 1, t.lane, wf);
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
  }
}

// Workgroup (b, y) computes rows [y rp, (y + 1) rp) of position b: gridDim.y
// is 1 (rp = N) up to BIG_MAX_N rows, 2 past it (GPW DMAs per chunk and wave
// then cover the position with three waves).
template <int EPI, int GPW = 9>
__global__ __launch_bounds__(256, 1) void hex_conv_big_kernel(const shrimp_conv_args a,
                                                              uint32_t x_bytes, uint32_t w_bytes,
                                                              int rp) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];
  SHRIMP_PHASE_WG(0);  // phase builds: the gather (row staging) starts
  BigParams<1> bp;
  bp.load(0, a.bias, a.ln_w, a.ln_b, (EPI & EPI_HEAD) ? a.head_w : a.gamma);
  BigTile t;
  const int rbase = (int)blockIdx.y * rp;
  big_setup<GPW>(t, a, xs, x_bytes, rbase, rbase + rp);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);
  u32x4 wf[8];
  big_wload(wr, 0, t.lane, wf);
  float* lp = reinterpret_cast<float*>(xs + 4 * t.NR * 64);
  bp.store(lp);
  // the accumulators start from the bias, except for the residual epilogue,
  // which adds it at the end like the fused ConvBlock's second conv (the two
  // give bit-identical blocks)
  constexpr int BA = (EPI & EPI_RESID) ? 0 : EPI_BACC;
  f32x4 acc[8][8];
  if constexpr (BA != 0) {
    big_acc_init(acc, a.bias, t.lg);
  } else {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  SHRIMP_PHASE_WG(1);  // phase builds: the position's rows are in LDS
  big_pass(acc, wf, t, xs, wr);
  SHRIMP_PHASE_WAVE(0);  // phase builds: this wave's epilogue starts
  if constexpr ((EPI & EPI_HEAD) != 0) {
    conv_epilogue<128, 8, EPI | BA, PS_LDS>(a, acc, t.rb, t.rn, t.rv, t.lg, lp);
  } else {
    conv_epilogue<128, 8, EPI | BA, PS_LDS>(a, acc, t.rb, t.rn, t.rv, t.lg, lp,
                                            GlobalRowStore16<8>(a, t.rb, t.rn, t.lg));
  }
  SHRIMP_PHASE_WAVE(1);  // phase builds: this wave's stores are issued
}

// Epilogue store of a ConvBlock that another ConvBlock follows in the same
// launch: every row goes to HBM (BufRowStore16: the next block's residual and
// the trunk state), and the rows that exist also into the LDS row layout as
// the next block's input (rows >= N are never written there: row N is the zero
// row).
struct BlockOutStore : BufRowStore16<8> {
  unsigned char* xs;
  uint32_t nr64;
  const BigTile& t;
  SHRIMP_DEV BlockOutStore(const shrimp_conv_args& a, const BigTile& tt, unsigned char* x, uint32_t o_bytes,
                           uint32_t r_bytes)
      : BufRowStore16<8>(a, tt.rb, tt.rn, tt.rv, tt.lg, o_bytes, r_bytes), xs(x),
        nr64((uint32_t)tt.NR * 64), t(tt) {}
  SHRIMP_DEV void operator()(int mb, int nb, u32x2 pk) {
    if (t.rv[mb]) {
      const uint32_t row = (uint32_t)t.rn[mb] * 64, swz = (uint32_t)((t.rn[mb] >> 2) & 3);
      const uint32_t piece = (uint32_t)((nb & 1) * 2 + (t.lg >> 1));
      *reinterpret_cast<u32x2*>(xs + (uint32_t)(nb >> 1) * nr64 + row + ((piece ^ swz) << 4) +
                                (uint32_t)(t.lg & 1) * 8) = pk;
    }
    BufRowStore16<8>::operator()(mb, nb, pk);
  }
};

// The two convs of one ConvBlock over the rows in LDS (ConvBlock.forward,
// model.py:395-422):
//   y1  = relu(LN1(conv1(x))) * m          -> written into LDS over x's rows
//   out = relu(x + gamma * LN2(conv2(y1)) * m)
// After a barrier conv1's epilogue writes y1 (bf16, masked rows zero) into the
// x layout and conv2 gathers from there, so y1 never reaches HBM; the zero row
// N stays zero. `c2.resid` is x and `c2.out` may alias it: a wave's residual
// reads of a row block complete before that block's stores (the stored values
// depend on them), and a wave only touches its own rows. NEXT: another block
// follows, and the output rows also become its input rows in LDS.
// first: x arrives by the DMA that big_setup issued (waited for here);
// otherwise the previous block wrote it into LDS.
template <bool NEXT>
SHRIMP_DEV void block_convs(BigTile& t, unsigned char* xs, const shrimp_conv_args& c1,
                            const shrimp_conv_args& a2, int pslot, uint32_t w_bytes,
                            uint32_t o_bytes, uint32_t r_bytes, bool first) {
  if (!first) {
    // as before conv2: the previous block's LDS row and weight offsets are
    // recomputed, not kept alive (spilled) for reuse
#pragma unroll
    for (int tp = 0; tp < 7; ++tp)
#pragma unroll
      for (int m2 = 0; m2 < 4; ++m2) asm volatile("" : "+v"(t.sw2[tp][m2]));
    asm volatile("" : "+v"(t.lane));
    t.lg = t.lane >> 4;
  }
  const __amdgpu_buffer_rsrc_t wr1 = make_rsrc(c1.w, w_bytes);
  const __amdgpu_buffer_rsrc_t wr2 = make_rsrc(a2.w, w_bytes);
  u32x4 wf[8];
  big_wload(wr1, 0, t.lane, wf);
  // this block's parameter sets: slots pslot and pslot + 1 after the rows
  const float* lp1 = reinterpret_cast<const float*>(xs + 4 * t.NR * 64) + pslot * BIG_PARAMS;
  const float* lp2 = lp1 + BIG_PARAMS;
  f32x4 acc[8][8];
  big_acc_init(acc, c1.bias, t.lg);
  // phase builds: workgroup stamps ps + 0..3 (ps = 1 for the first block of a
  // pair, 5 for the second), per-wave stamps at the last block's epilogue
  const int ps = first ? 1 : 5;
  (void)ps;
  if (first) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  } else {
    // the previous block's LDS writes are complete (its HBM stores need not be)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  }
  SHRIMP_PHASE_WG(ps);  // rows in LDS: conv1 starts
  // conv2's first weights are loaded after conv1's epilogue, whose bias and
  // ln_w then fit in registers
  big_pass(acc, wf, t, xs, wr1);
  __syncthreads();  // every wave is done reading x from LDS
  SHRIMP_PHASE_WG(ps + 1);  // epilogue 1 starts
  {
    const uint32_t nr64 = (uint32_t)t.NR * 64;
    const uint32_t lo = (uint32_t)(t.lg & 1) * 8;
    uint32_t row[8], swz[8];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      row[mb] = (uint32_t)t.rn[mb] * 64;
      swz[mb] = (uint32_t)((t.rn[mb] >> 2) & 3);
    }
    const int lg = t.lg;
    big_rows(t);
    conv_epilogue<128, 8, EPI_LN | EPI_RELU | EPI_BACC, PS_LDSREG>(
        c1, acc, t.rb, t.rn, t.rv, t.lg, lp1, [&](int mb, int nb, u32x2 pk) {
          const uint32_t piece = (uint32_t)((nb & 1) * 2 + (lg >> 1));
          const uint32_t addr = (uint32_t)(nb >> 1) * nr64 + row[mb] + ((piece ^ swz[mb]) << 4) + lo;
          *reinterpret_cast<u32x2*>(xs + addr) = pk;
        });
  }
  // conv2 starts from zeros and adds its bias in the epilogue: starting from
  // the bias here makes the register allocator spill
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // y1 is complete
  SHRIMP_PHASE_WG(ps + 2);  // conv2 starts
  big_wload(wr2, 0, t.lane, wf);
  // Hide the per-lane addresses from the optimizer: otherwise it keeps conv1's
  // LDS row and weight offsets alive (spilled) for reuse by conv2 instead of
  // recomputing them.
#pragma unroll
  for (int tp = 0; tp < 7; ++tp)
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) asm volatile("" : "+v"(t.sw2[tp][m2]));
  asm volatile("" : "+v"(t.lane));
  t.lg = t.lane >> 4;
  big_pass(acc, wf, t, xs, wr2);
  if constexpr (NEXT) {
    // every wave is done reading y1 before the output rows replace it
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    SHRIMP_PHASE_WG(ps + 3);  // epilogue 2 (residual reads, row stores) starts
    big_rows(t);
    conv_epilogue<128, 8, EPI_LN | EPI_RESID, PS_LDS>(a2, acc, t.rb, t.rn, t.rv, t.lg, lp2,
                                                      BlockOutStore(a2, t, xs, o_bytes, r_bytes));
  } else {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) asm volatile("" : "+a"(acc[nb][mb]));
    SHRIMP_PHASE_WAVE(0);  // this wave's epilogue 2 starts
    big_rows(t);
    conv_epilogue<128, 8, EPI_LN | EPI_RESID, PS_LDS>(
        a2, acc, t.rb, t.rn, t.rv, t.lg, lp2,
        BufRowStore16<8>(a2, t.rb, t.rn, t.rv, t.lg, o_bytes, r_bytes));
    SHRIMP_PHASE_WAVE(1);  // this wave's stores are issued
  }
}

// ConvBlock in one launch (ConvBlock.forward, model.py:395-422):
//   y1  = relu(LN1(conv1(x))) * m          -> written into LDS over x's rows
//   out = relu(x + gamma * LN2(conv2(y1)) * m)
// conv1 stages x and runs as the big-tile conv; after a barrier its epilogue
// writes y1 (bf16, masked rows zero) into the same LDS layout, and conv2
// gathers from there, so y1 never reaches HBM. The zero row N stays zero.
// `c2.resid` is x and `c2.out` may alias it: a wave's residual reads of a row
// block complete before that block's stores (the stored values depend on
// them), and a wave only touches its own rows.
__global__ __launch_bounds__(256, 1) void hex_block_kernel(const shrimp_conv_args c1,
                                                           const shrimp_conv_args c2,
                                                           uint32_t x_bytes, uint32_t w_bytes,
                                                           uint32_t o_bytes) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];
  BigParams<2> bp;
  bp.load(0, c1.bias, c1.ln_w, c1.ln_b, nullptr);
  bp.load(1, c2.bias, c2.ln_w, c2.ln_b, c2.gamma);
  BigTile t;
  big_setup(t, c1, xs, x_bytes);
  const __amdgpu_buffer_rsrc_t wr1 = make_rsrc(c1.w, w_bytes);
  const __amdgpu_buffer_rsrc_t wr2 = make_rsrc(c2.w, w_bytes);
  u32x4 wf[8];
  big_wload(wr1, 0, t.lane, wf);
  float* lp1 = reinterpret_cast<float*>(xs + 4 * t.NR * 64);
  float* lp2 = lp1 + BIG_PARAMS;
  bp.store(lp1);
  f32x4 acc[8][8];
  big_acc_init(acc, c1.bias, t.lg);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // conv2's first weights are loaded after conv1's epilogue, whose bias and
  // ln_w then fit in registers
  big_pass(acc, wf, t, xs, wr1);
  __syncthreads();  // every wave is done reading x from LDS
  {
    const uint32_t nr64 = (uint32_t)t.NR * 64;
    const uint32_t lo = (uint32_t)(t.lg & 1) * 8;
    uint32_t row[8], swz[8];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      row[mb] = (uint32_t)t.rn[mb] * 64;
      swz[mb] = (uint32_t)((t.rn[mb] >> 2) & 3);
    }
    const int lg = t.lg;
    conv_epilogue<128, 8, EPI_LN | EPI_RELU | EPI_BACC, PS_LDSREG>(
        c1, acc, t.rb, t.rn, t.rv, t.lg, lp1, [&](int mb, int nb, u32x2 pk) {
          const uint32_t piece = (uint32_t)((nb & 1) * 2 + (lg >> 1));
          const uint32_t addr = (uint32_t)(nb >> 1) * nr64 + row[mb] + ((piece ^ swz[mb]) << 4) + lo;
          *reinterpret_cast<u32x2*>(xs + addr) = pk;
        });
  }
  // conv2 starts from zeros and adds its bias in the epilogue: starting from
  // the bias here makes the register allocator spill
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // y1 is complete
  big_wload(wr2, 0, t.lane, wf);
  // Hide the per-lane addresses from the optimizer: otherwise it keeps conv1's
  // LDS row and weight offsets alive (spilled) for reuse by conv2 instead of
  // recomputing them.
#pragma unroll
  for (int tp = 0; tp < 7; ++tp)
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) asm volatile("" : "+v"(t.sw2[tp][m2]));
  asm volatile("" : "+v"(t.lane));
  t.lg = t.lane >> 4;
  big_pass(acc, wf, t, xs, wr2);
  conv_epilogue<128, 8, EPI_LN | EPI_RESID, PS_LDS>(
      c2, acc, t.rb, t.rn, t.rv, t.lg, lp2,
      BufRowStore16<8>(c2, t.rb, t.rn, t.rv, t.lg, o_bytes, x_bytes));
}

// What the second ConvBlock of a pair needs beyond the first one's arguments:
// its weights, epsilons and epilogue parameters (it reads and writes the
// first block's output rows, with the first block's index, mask and shape).
struct PairSecond {
  const void* w3;
  const float* b3;
  const float* l3w;
  const float* l3b;
  float eps3;
  const void* w4;
  const float* b4;
  const float* l4w;
  const float* l4b;
  const float* g4;
  float eps4;
};

// Two consecutive ConvBlocks in one launch: x staged once by DMA
// (big_setup), the first block's output rows handed to the second in LDS, so
// the second does not read them back from HBM for its convs (its residual
// reads them: a wave reads rows it wrote itself, and writes them again in
// place). x_bytes spans c1.x (the first residual), o_bytes c2.out (the second
// block's residual and output).
__global__ __launch_bounds__(256, 1) void hex_block_pair_kernel(
    const shrimp_conv_args c1, const shrimp_conv_args c2, const PairSecond p2, uint32_t x_bytes,
    uint32_t w_bytes, uint32_t o_bytes) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];
  SHRIMP_PHASE_WG(0);  // phase builds: the gather (row staging) starts
  BigParams<4> bp;
  bp.load(0, c1.bias, c1.ln_w, c1.ln_b, nullptr);
  bp.load(1, c2.bias, c2.ln_w, c2.ln_b, c2.gamma);
  bp.load(2, p2.b3, p2.l3w, p2.l3b, nullptr);
  bp.load(3, p2.b4, p2.l4w, p2.l4b, p2.g4);
  BigTile t;
  big_setup(t, c1, xs, x_bytes);
  bp.store(reinterpret_cast<float*>(xs + 4 * t.NR * 64));
  block_convs<true>(t, xs, c1, c2, 0, w_bytes, o_bytes, x_bytes, true);
  shrimp_conv_args c3 = c1;
  c3.w = p2.w3;
  c3.bias = p2.b3;
  c3.eps = p2.eps3;
  shrimp_conv_args c4 = c2;
  c4.w = p2.w4;
  c4.eps = p2.eps4;
  c4.resid = c2.out;
  c4.r_sb = c2.o_sb;
  c4.r_sn = c2.o_sn;
  block_convs<false>(t, xs, c3, c4, 2, w_bytes, o_bytes, o_bytes, false);
}

// ---- trunk tail + policy head (model.py:927-935, 990-1020) ---------------------
// The final LayerNorm of shrimp_trunk_tail's first pass (final_ln_kernel) with
// the same arithmetic and summation order, over one position: its cell rows
// in place in LDS (the big-tile conv's row layout, staged by big_setup), token
// rows 0, 1, 4 and 5 from seq; the head inputs [T0 | T1 | pooled | T4 | T5 |
// pooled] to the workspace. As in final_ln_kernel a row is 16 lanes of 8
// channels, and row slot rs (= row % 16) pools its cells in row order; the 16
// slot sums then add in slot order (red: [16][128] floats, cred: [16]). mk:
// the position's cell mask bytes, staged in LDS.
SHRIMP_DEV void tail_ln_lds(const BigTile& t, unsigned char* xs, const shrimp_tail_args& ta,
                            float* red, float* cred, const uint8_t* mk) {
  constexpr int C = 128;
  const int S = ta.S, nt = ta.n_tokens;
  const int tid = threadIdx.x, ngrp = (int)(blockDim.x >> 4);
  const int sub = tid & 15, c0 = sub * 8;
  const uint32_t koff = (uint32_t)((sub >> 2) * t.NR * 64), piece = (uint32_t)(sub & 3);
  const uint16_t* seq = static_cast<const uint16_t*>(ta.seq) + (int64_t)t.b * ta.s_sb;
  const uint16_t* tlo =
      ta.tok_lo ? static_cast<const uint16_t*>(ta.tok_lo) + (int64_t)t.b * nt * C : nullptr;
  float* vin = ta.workspace + (int64_t)t.b * 6 * C;
  float w[8], bb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = ta.ln_w[c0 + e];
    bb[e] = ta.ln_b[c0 + e];
  }
  const float invc = 1.0f / (float)C;
  // One row: x = raw + lo (the low part of a token row, zeros for a cell row:
  // final_ln_kernel adds it the same way), normalised into y (zeros where not
  // live).
  auto norm_row = [&](const u32x4& raw, const u32x4& lo, bool live, float (&y)[8]) {
    float x[8];
    float sm = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf16_lo(raw[e]) + bf16_lo(lo[e]);
      x[2 * e + 1] = bf16_hi(raw[e]) + bf16_hi(lo[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) sm += x[e];
    sm = group_sum_dpp<16>(sm);
    const float mean = sm * invc;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = x[e] - mean;
      q = fmaf(x[e], x[e], q);
    }
    q = group_sum_dpp<16>(q);
    const float rstd = rsqrtf(q * invc + ta.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = live ? fmaf(x[e] * rstd, w[e], bb[e]) : 0.f;
  };
  for (int rs = tid >> 4; rs < 16; rs += ngrp) {
    float pool[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pool[e] = 0.f;
    int cnt = 0;
    // Token rows (r < nt) from global memory, then the cell rows from LDS, in
    // row order. Two loops, so the cell rows are plain LDS reads: one loop
    // over both kinds compiled to a flat load through a selected pointer,
    // which gave every LDS row the global-memory latency.
    int r = rs;
    for (; r < nt && r < S; r += 16) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(seq + (int64_t)r * C + c0);
      const u32x4 lo = tlo ? *reinterpret_cast<const u32x4*>(tlo + (int64_t)r * C + c0)
                           : u32x4{0u, 0u, 0u, 0u};
      float y[8];
      norm_row(raw, lo, true, y);
      const int slot = r == 0 ? 0 : r == 1 ? 1 : r == 4 ? 3 : r == 5 ? 4 : -1;
      if (slot >= 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vin[slot * C + c0 + e] = y[e];
      }
    }
    for (; r < S; r += 16) {
      const int j = r - nt;
      const uint32_t addr = koff + (uint32_t)j * 64 + ((piece ^ (uint32_t)((j >> 2) & 3)) << 4);
      const u32x4 raw = *reinterpret_cast<const u32x4*>(xs + addr);
      const bool live = mk[j] != 0;
      float y[8];
      norm_row(raw, u32x4{0u, 0u, 0u, 0u}, live, y);
      *reinterpret_cast<u32x4*>(xs + addr) =
          u32x4{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                pack_bf16x2(y[6], y[7])};
      if (live && sub == 0) ++cnt;
#pragma unroll
      for (int e = 0; e < 8; ++e) pool[e] += y[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) red[rs * C + c0 + e] = pool[e];
    if (sub == 0) cred[rs] = (float)cnt;
  }
  __syncthreads();
  float total = 0.f;
  for (int i = 0; i < 16; ++i) total += cred[i];
  const float inv = 1.0f / fmaxf(1.f, total);
  for (int c = tid; c < C; c += (int)blockDim.x) {
    float p = 0.f;
    for (int i = 0; i < 16; ++i) p += red[i * C + c];
    vin[2 * C + c] = p * inv;
    vin[5 * C + c] = p * inv;
  }
}

// shrimp_policy_tail's first launch: the big-tile policy conv (conv + bias +
// ReLU + Linear(C, 1) head + mask, EPI_HEAD | EPI_RELU) whose staged rows are
// the position's pre-LayerNorm cells; tail_ln_lds normalises them in LDS first.
__global__ __launch_bounds__(256, 1) void policy_tail_kernel(const shrimp_conv_args a,
                                                             const shrimp_tail_args ta,
                                                             uint32_t x_bytes, uint32_t w_bytes) {
  constexpr int EPI = EPI_HEAD | EPI_RELU;
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];
  BigParams<1> bp;
  bp.load(0, a.bias, a.ln_w, a.ln_b, a.head_w);
  BigTile t;
  big_setup(t, a, xs, x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, w_bytes);
  u32x4 wf[8];
  big_wload(wr, 0, t.lane, wf);
  float* lp = reinterpret_cast<float*>(xs + 4 * t.NR * 64);
  float* red = lp + BIG_PARAMS;
  float* cred = red + 16 * 128;
  uint8_t* mk = reinterpret_cast<uint8_t*>(cred + 16);
  bp.store(lp);
  for (int j = threadIdx.x; j < t.N; j += blockDim.x) mk[j] = ta.mask[(int64_t)t.b * t.N + j];
  f32x4 acc[8][8];
  big_acc_init(acc, a.bias, t.lg);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  tail_ln_lds(t, xs, ta, red, cred, mk);
  __syncthreads();  // the normalised rows are complete
  big_pass(acc, wf, t, xs, wr);
  conv_epilogue<128, 8, EPI | EPI_BACC, PS_LDS>(a, acc, t.rb, t.rn, t.rv, t.lg, lp);
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
  const bool out16 = (EPI & EPI_HEAD) != 0 ||
                     (a->o_sn % 8 == 0 && a->o_sb % 8 == 0 && ((uintptr_t)a->out & 15) == 0);
  const size_t big_lds = (size_t)big_rows_padded(a->N) * 256 + BIG_PARAMS * sizeof(float);
  const bool big = COUT == 128 && lds && a->cin_pad == 128 && a->taps == 7 && a->N <= BIG_MAX_N &&
                   out16 && (g_conv_variant == 0 || g_conv_variant == 3) &&
                   big_lds <= (size_t)max_lds_per_block();
  // The LDS kernels keep the rows plus the per-channel parameters in LDS;
  // their 16-byte buffered stores (COUT = 128) need 16-byte aligned rows and
  // extents within the 32-bit buffer offsets.
  const size_t lds_p = lds ? ((lds + 15) & ~(size_t)15) + (size_t)5 * COUT * sizeof(float) : 0;
  const bool lds_ok = lds && lds_p <= (size_t)max_lds_per_block();
  const bool head = (EPI & EPI_HEAD) != 0;
  const int64_t o_ext = head ? 0 : ((int64_t)(a->B - 1) * a->o_sb + (int64_t)(a->N - 1) * a->o_sn + COUT) * 2;
  const int64_t r_ext =
      (EPI & EPI_RESID) ? ((int64_t)(a->B - 1) * a->r_sb + (int64_t)(a->N - 1) * a->r_sn + COUT) * 2 : 0;
  const bool b16 = COUT == 128 && !head && out16 && o_ext < (int64_t)0x7FFF0000 &&
                   r_ext < (int64_t)0x7FFF0000 &&
                   (!(EPI & EPI_RESID) || (a->r_sn % 4 == 0 && a->r_sb % 4 == 0));
  const uint32_t ob = (uint32_t)o_ext, rbb = (uint32_t)r_ext;
#define SHRIMP_LDS_LAUNCH(GRID, MBV, CINV, BIGO)                                                     \
  do {                                                                                             \
    if (b16)                                                                                       \
      hipLaunchKernelGGL((hex_conv_lds_kernel<COUT, MBV, EPI, CINV, BIGO, COUT == 128>), GRID,     \
                         dim3(256), lds_p, st, *a, wb, ob, rbb);                                   \
    else                                                                                           \
      hipLaunchKernelGGL((hex_conv_lds_kernel<COUT, MBV, EPI, CINV, BIGO, false>), GRID, dim3(256), \
                         lds_p, st, *a, wb, ob, rbb);                                              \
    return check_launch("hex_conv");                                                               \
  } while (0)
  // Past BIG_MAX_N rows a position's rows split over two workgroups of three
  // waves (rows [0, rp) and [rp, N), rp = ceil(N / 32) * 16), each staging the
  // whole position: the big-tile arithmetic (same bits per row) with one
  // round of workgroups for up to a compute unit's worth of halves, where the
  // row-split kernel stages the position once per 64-row tile. Batches under
  // BIG_SPLIT_MIN_B positions keep the row split (more workgroups).
  if (COUT == 128 && lds && a->cin_pad == 128 && a->taps == 7 && a->N > BIG_MAX_N &&
      a->B >= BIG_SPLIT_MIN_B &&
      a->N <= BIG_SPLIT_MAX_N && out16 && (g_conv_variant == 0 || g_conv_variant == 3) &&
      big_lds <= (size_t)max_lds_per_block()) {
    const int rp = (a->N + 31) / 32 * 16;
    hipLaunchKernelGGL((hex_conv_big_kernel<EPI, BIG_SPLIT_GPW>), dim3(a->B, 2), dim3(64 * 3),
                       big_lds, st, *a, xb, wb, rp);
    return check_launch("hex_conv");
  }
  // Small batches (at most half as many positions as compute units): one row
  // tile of 64 rows per workgroup, (B, N / 64) workgroups, instead of one
  // workgroup per position; where the big-tile kernel would run, with its
  // arithmetic (same bits).
  // (The big-tile order adds a static 16 * COUT-byte weight buffer to the LDS.)
  if (COUT == 128 && lds_ok && (a->cin_pad == 32 || a->cin_pad == 128) &&
      (int64_t)a->B * 2 <= cu_count() && g_conv_variant == 0 &&
      (!big || lds_p + (size_t)COUT * 64 <= (size_t)max_lds_per_block())) {
    const dim3 grid((unsigned)a->B, (unsigned)((a->N + 63) / 64));
    if (big) SHRIMP_LDS_LAUNCH(grid, 1, 128, true);
    else if (a->cin_pad == 32) SHRIMP_LDS_LAUNCH(grid, 1, 32, false);
    else SHRIMP_LDS_LAUNCH(grid, 1, 128, false);
  }
  if (big) {
    const int waves = (a->N + 127) / 128;
    {
      hipLaunchKernelGGL((hex_conv_big_kernel<EPI>), dim3(a->B), dim3(64 * waves), big_lds, st, *a,
                         xb, wb, a->N);
      return check_launch("hex_conv");
    }
  }

  if (lds_ok) {
    switch (a->cin_pad) {
      case 32: SHRIMP_LDS_LAUNCH(dim3(a->B), MB, 32, false);
      case 64: SHRIMP_LDS_LAUNCH(dim3(a->B), MB, 64, false);
      case 128: SHRIMP_LDS_LAUNCH(dim3(a->B), MB, 128, false);
      default:
        break;
    }
  }
#undef SHRIMP_LDS_LAUNCH
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

// 0 for a shape whose packed weights would not fit a 32-bit buffer offset
extern "C" size_t shrimp_conv_wpack_bytes(int taps, int cin_pad, int cout) {
  const int64_t n = mul_sat({taps, cin_pad, cout, 2});
  return taps > 0 && cin_pad > 0 && cout > 0 && n < (int64_t)0x7FFF0000 ? (size_t)n : 0;
}

extern "C" size_t shrimp_linear_wpack_bytes(int in_features, int out_features) {
  const int64_t n = mul_sat({in_features, out_features, 2});
  return in_features > 0 && out_features > 0 && n < (int64_t)0x7FFF0000 ? (size_t)n : 0;
}

extern "C" int shrimp_phase_clock(void* stamps, int unit) {
  SHRIMP_REQUIRE(unit >= 0 && unit <= 5 && (unit & 3) <= 1,
                 "phase_clock: unit %d (0 conv kernels, 1 attention, + 4 for the core clock)", unit);
  const int cycles = unit & 4;
  if ((unit & 3) == 1) return attn_phase_set(stamps, cycles);
#if SHRIMP_PHASE_CLOCK
  return phase_set(stamps, cycles);
#else
  (void)cycles;
  (void)stamps;
  return set_error(SHRIMP_EINVAL, "phase_clock: phase stamps need the phase build (SHRIMP_PHASE_CLOCK=1)");
#endif
}

extern "C" int shrimp_pack_conv_weight(const float* w, void* packed, int taps, int cin,
                                       int cin_pad, int cout, void* stream) {
  SHRIMP_REQUIRE(w && packed, "pack_conv_weight: null pointer");
  SHRIMP_REQUIRE(taps > 0 && cin > 0 && cin <= cin_pad && cin_pad % 32 == 0,
                 "pack_conv_weight: bad taps/cin (%d, %d, %d)", taps, cin, cin_pad);
  SHRIMP_REQUIRE(cout > 0 && cout % 16 == 0, "pack_conv_weight: cout %d not a multiple of 16",
                 cout);
  SHRIMP_REQUIRE(shrimp_conv_wpack_bytes(taps, cin_pad, cout) > 0, "pack_conv_weight: too large");
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
  SHRIMP_REQUIRE(in_features % 32 == 0 && out_features % 16 == 0 &&
                     shrimp_linear_wpack_bytes(in_features, out_features) > 0,
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
  SHRIMP_REQUIRE(a->B >= 0 && a->N > 0 && a->N <= kMaxDim, "hex_conv: bad B/N (%d, %d)", a->B, a->N);
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->idx && a->mask && a->w && a->bias, "hex_conv: null input pointer");
  SHRIMP_REQUIRE(a->taps > 0 && a->idx_stride >= a->taps, "hex_conv: bad taps %d / stride %d",
                 a->taps, a->idx_stride);
  SHRIMP_REQUIRE(a->cin_pad > 0 && a->cin_pad % 32 == 0, "hex_conv: cin_pad %d %% 32 != 0",
                 a->cin_pad);
  SHRIMP_REQUIRE(strides_ok({a->x_sb, a->x_sn, a->o_sb, a->o_sn, a->r_sb, a->r_sn}),
                 "hex_conv: strides outside [0, 2^31)");
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

extern "C" int shrimp_conv_block_supported(int taps, int N, int cin_pad, int cout) {
  if (taps != 7 || cin_pad != 128 || cout != 128 || N <= 0 || N > BIG_MAX_N) return 0;
  if (g_conv_variant != 0 && g_conv_variant != 3) return 0;
  const size_t lds = (size_t)big_rows_padded(N) * 256 + 2 * BIG_PARAMS * sizeof(float);
  return lds <= (size_t)max_lds_per_block() ? 1 : 0;
}

// Checks of one ConvBlock's two conv argument sets (the contract of
// shrimp_conv_block); fills conv2's launch arguments (x, index, mask and shape
// of conv1) and the byte extents of x and of the output.
static int check_block(const shrimp_conv_args* c1, const shrimp_conv_args* c2, shrimp_conv_args* a2_out,
                       int64_t* x_bytes, int64_t* o_bytes) {
  SHRIMP_REQUIRE(c1 != nullptr && c2 != nullptr, "conv_block: null args");
  SHRIMP_REQUIRE(c1->B >= 0 && c1->N > 0, "conv_block: bad B/N (%d, %d)", c1->B, c1->N);
  SHRIMP_REQUIRE(shrimp_conv_block_supported(c1->taps, c1->N, c1->cin_pad, c1->cout) &&
                     c2->cin_pad == 128 && c2->cout == 128,
                 "conv_block: no fused kernel for taps %d, N %d, %d -> %d channels", c1->taps,
                 c1->N, c1->cin_pad, c1->cout);
  SHRIMP_REQUIRE(c1->x && c1->idx && c1->mask && c1->w && c1->bias && c2->w && c2->bias,
                 "conv_block: null input pointer");
  SHRIMP_REQUIRE(c1->idx_stride >= 7, "conv_block: idx_stride %d < 7", c1->idx_stride);
  SHRIMP_REQUIRE(strides_ok({c1->x_sb, c1->x_sn, c2->o_sb, c2->o_sn}), "conv_block: strides outside [0, 2^31)");
  SHRIMP_REQUIRE(c1->ln_w && c1->ln_b && c1->relu && !c1->resid && !c1->head_w,
                 "conv_block: conv1 must be conv + LN + ReLU");
  SHRIMP_REQUIRE(c2->ln_w && c2->ln_b && !c2->relu && c2->gamma && !c2->head_w && c2->out,
                 "conv_block: conv2 must be conv + LN + LayerScale residual");
  SHRIMP_REQUIRE(c2->resid == c1->x && c2->r_sb == c1->x_sb && c2->r_sn == c1->x_sn,
                 "conv_block: the residual must be the block input");
  SHRIMP_REQUIRE((reinterpret_cast<uintptr_t>(c1->x) & 15) == 0 && c1->x_sn >= 128 &&
                     c1->x_sn % 8 == 0 && c1->x_sb % 8 == 0,
                 "conv_block: x rows must be 16-byte aligned");
  SHRIMP_REQUIRE(c2->o_sn % 8 == 0 && c2->o_sb % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(c2->out) & 15) == 0,
                 "conv_block: output rows must be 16-byte aligned (strides %% 8)");
  const int64_t x_extent =
      (int64_t)(c1->B - 1) * c1->x_sb + (int64_t)(c1->N - 1) * c1->x_sn + c1->cin_pad;
  SHRIMP_REQUIRE(x_extent * 2 < (int64_t)0x7FFF0000, "conv_block: activation buffer too large");
  shrimp_conv_args a2 = *c2;
  a2.x = c1->x;
  a2.x_sb = c1->x_sb;
  a2.x_sn = c1->x_sn;
  a2.idx = c1->idx;
  a2.taps = 7;
  a2.idx_stride = c1->idx_stride;
  a2.mask = c1->mask;
  a2.B = c1->B;
  a2.N = c1->N;
  const int64_t o_extent =
      (int64_t)(c1->B - 1) * c2->o_sb + (int64_t)(c1->N - 1) * c2->o_sn + 128;
  SHRIMP_REQUIRE(o_extent * 2 < (int64_t)0x7FFF0000, "conv_block: output buffer too large");
  *a2_out = a2;
  *x_bytes = x_extent * 2;
  *o_bytes = o_extent * 2;
  return SHRIMP_OK;
}

extern "C" int shrimp_conv_block(const shrimp_conv_args* c1, const shrimp_conv_args* c2,
                                 void* stream) {
  SHRIMP_REQUIRE(c1 != nullptr && c2 != nullptr, "conv_block: null args");
  if (c1->B == 0) return SHRIMP_OK;
  shrimp_conv_args a2;
  int64_t xb = 0, ob = 0;
  if (int rc = check_block(c1, c2, &a2, &xb, &ob)) return rc;
  const int waves = (c1->N + 127) / 128;
  const size_t lds = (size_t)big_rows_padded(c1->N) * 256 + 2 * BIG_PARAMS * sizeof(float);
  const uint32_t wb = (uint32_t)shrimp_conv_wpack_bytes(7, 128, 128);
  hipLaunchKernelGGL(hex_block_kernel, dim3(c1->B), dim3(64 * waves), lds, as_stream(stream), *c1,
                     a2, (uint32_t)xb, wb, (uint32_t)ob);
  return check_launch("conv_block");
}

static size_t block_pair_lds(int N) {
  return (size_t)big_rows_padded(N) * 256 + 4 * BIG_PARAMS * sizeof(float);
}

extern "C" int shrimp_conv_block_pair_supported(int taps, int N, int cin_pad, int cout) {
  return shrimp_conv_block_supported(taps, N, cin_pad, cout) &&
         block_pair_lds(N) <= (size_t)max_lds_per_block();
}

extern "C" int shrimp_conv_block_pair(const shrimp_conv_args* c1, const shrimp_conv_args* c2,
                                      const shrimp_conv_args* c3, const shrimp_conv_args* c4,
                                      void* stream) {
  SHRIMP_REQUIRE(c1 && c2 && c3 && c4, "conv_block_pair: null args");
  if (c1->B == 0) return SHRIMP_OK;
  shrimp_conv_args a2, a4;
  int64_t xb = 0, ob = 0, xb3 = 0, ob4 = 0;
  if (int rc = check_block(c1, c2, &a2, &xb, &ob)) return rc;
  if (int rc = check_block(c3, c4, &a4, &xb3, &ob4)) return rc;
  SHRIMP_REQUIRE(c3->x == c2->out && c3->x_sb == c2->o_sb && c3->x_sn == c2->o_sn,
                 "conv_block_pair: the second block's input must be the first block's output");
  SHRIMP_REQUIRE(c3->idx == c1->idx && c3->idx_stride == c1->idx_stride && c3->mask == c1->mask &&
                     c3->B == c1->B && c3->N == c1->N,
                 "conv_block_pair: both blocks must share the index, mask and shape");
  SHRIMP_REQUIRE(c4->out == c2->out && c4->o_sb == c2->o_sb && c4->o_sn == c2->o_sn,
                 "conv_block_pair: the second block must write in place over the first block's output");
  SHRIMP_REQUIRE(shrimp_conv_block_pair_supported(7, c1->N, 128, 128),
                 "conv_block_pair: %d rows do not fit the LDS of one workgroup", c1->N);
  const int waves = (c1->N + 127) / 128;
  const uint32_t wb = (uint32_t)shrimp_conv_wpack_bytes(7, 128, 128);
  const PairSecond p2{c3->w, c3->bias, c3->ln_w, c3->ln_b, c3->eps,
                      c4->w, c4->bias, c4->ln_w, c4->ln_b, c4->gamma, c4->eps};
  hipLaunchKernelGGL(hex_block_pair_kernel, dim3(c1->B), dim3(64 * waves), block_pair_lds(c1->N),
                     as_stream(stream), *c1, a2, p2, (uint32_t)xb, wb, (uint32_t)ob);
  return check_launch("conv_block_pair");
}

static size_t policy_tail_lds(int N) {
  return (size_t)big_rows_padded(N) * 256 + (BIG_PARAMS + 16 * 128 + 16) * sizeof(float) +
         (size_t)((N + 15) & ~15);
}

extern "C" int shrimp_policy_tail_supported(int N, int C) {
  return C == 128 && N > 0 && N <= BIG_MAX_N && (g_conv_variant == 0 || g_conv_variant == 3) &&
         policy_tail_lds(N) <= (size_t)max_lds_per_block();
}

extern "C" int shrimp_policy_tail(const shrimp_conv_args* p, const shrimp_tail_args* ta,
                                  void* stream) {
  SHRIMP_REQUIRE(p != nullptr && ta != nullptr, "policy_tail: null args");
  if (ta->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(ta->seq && ta->mask && ta->ln_w && ta->ln_b && ta->workspace,
                 "policy_tail: null tail pointer");
  SHRIMP_REQUIRE(ta->C == 128 && ta->n_tokens >= 6 && ta->S > ta->n_tokens && ta->s_sb % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(ta->seq) & 15) == 0,
                 "policy_tail: needs C = 128, >= 6 tokens, 16-byte aligned rows (C %d, tokens %d)",
                 ta->C, ta->n_tokens);
  SHRIMP_REQUIRE(!ta->value || (ta->vr_w && ta->vr_b && ta->vh_w && ta->vh_b),
                 "policy_tail: value head");
  SHRIMP_REQUIRE(!ta->moves_left || (ta->mr_w && ta->mr_b && ta->mh_w && ta->mh_b),
                 "policy_tail: moves-left head");
  SHRIMP_REQUIRE(ta->bins > 0 && ta->bins <= 256, "policy_tail: bins %d", ta->bins);
  const int N = ta->S - ta->n_tokens;
  SHRIMP_REQUIRE(shrimp_policy_tail_supported(N, ta->C), "policy_tail: no fused kernel for N %d", N);
  SHRIMP_REQUIRE(p->B == ta->B && p->N == N && p->cin_pad == 128 && p->cout == 128 && p->taps == 7 &&
                     p->idx_stride >= 7 && p->idx && p->w && p->bias && p->head_w && p->head_b &&
                     p->head_out && p->relu && !p->ln_w && !p->resid,
                 "policy_tail: policy must be the 7-tap 128-channel conv + ReLU + head over the cells");
  SHRIMP_REQUIRE(p->x == static_cast<const uint16_t*>(ta->seq) + (int64_t)ta->n_tokens * 128 &&
                     p->x_sb == ta->s_sb && p->x_sn == 128 && p->mask == ta->mask,
                 "policy_tail: the policy conv must read the cell rows of tail.seq with its mask");
  SHRIMP_REQUIRE(strides_ok({p->x_sb}), "policy_tail: position stride outside [0, 2^31)");
  const int64_t x_extent = (int64_t)(p->B - 1) * p->x_sb + (int64_t)(N - 1) * p->x_sn + 128;
  SHRIMP_REQUIRE(x_extent * 2 < (int64_t)0x7FFF0000, "policy_tail: activation buffer too large");
  const int waves = (N + 127) / 128;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(policy_tail_kernel, dim3(p->B), dim3(64 * waves), policy_tail_lds(N), st, *p,
                     *ta, (uint32_t)(x_extent * 2), (uint32_t)shrimp_conv_wpack_bytes(7, 128, 128));
  if (int rc = check_launch("policy_tail")) return rc;
  return launch_value_heads(ta, st);
}
