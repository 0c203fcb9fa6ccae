// hexfield_eq serve kernels on the 32-slot ray gather index, gfx950.
//
//  * ray_attn_kernel: hexfield_eq::ray_attn
//    (packages/hexfield_eq/python/hexfield_eq/_triton_ray.py:378-501, op
//    :681-715). Each query row attends to at most 11 keys: itself (slot 0) and
//    the ten cells of its head's win axis (slots 1 + axis*10 + dir*5 + k-1)
//    whose step k is within the ray's reach. A workgroup takes one position
//    and one head pair (heads 2p, 2p+1 share the axis, hence the index slots
//    and the key rows); the pair's K and V rows are staged in LDS when they
//    fit and every query gathers its keys from there. Only live slots are
//    fetched: dead slots carry exactly zero weight in the reference's fp32
//    softmax (score -3e4 against a live score).
//  * conv_ln_raytap_kernel: hexfield_eq::hex_conv_ln_raytap, K1
//    (_triton_conv.py:391-499, op :501-555). One workgroup per position,
//    x rows staged in LDS with a zero row at N. Tap 0 is the centre row; taps
//    1..6 are built per lane as the fp16 MFMA operand: five ray rows summed in
//    fp32 with their alpha weights. Visibility (k <= reach of the channel's
//    side) is applied through the address: an invisible step reads the zero
//    row, for each 4-channel half of the lane's 8 channels separately (each
//    half lies on one side when corb % 8 == 0). Product on
//    v_mfma_f32_16x16x32_f16 in the transposed orientation out^T = W^T X^T, then
//    LayerNorm over the output channels inside the wave.
#include "capi.hpp"
#include "common.hpp"

typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

namespace {

using namespace shrimp;

constexpr int RAY_SLOT_COUNT = 32;
constexpr int RAY_STEPS = 5;
constexpr int RA_THREADS = 256;
constexpr uint32_t RA_STAGE_MAX_LDS = 64 * 1024;
constexpr uint32_t RA_BIAS_LDS = 96;  // the head pair's 22 fp32 slot biases, padded
constexpr float LOG2E_F = 1.4426950408889634f;

std::atomic<int> g_ray_variant{0};

SHRIMP_DEV f16x2 as_h2(unsigned u) { return __builtin_bit_cast(f16x2, u); }

SHRIMP_DEV unsigned pack_f16x2(float lo, float hi) {
  f16x2 h;
  h.x = (_Float16)lo;
  h.y = (_Float16)hi;
  return __builtin_bit_cast(unsigned, h);
}

template <int D>
constexpr float inv_sqrt_d() {
  return D == 16 ? 0.25f : D == 32 ? 0.17677669529663687f : D == 64 ? 0.125f : 0.08838834764831845f;
}

// ---- ray attention ---------------------------------------------------------------

// 16 fp16 of a row (two 16-byte pieces).
struct Row16 {
  u32x4 p0, p1;
};

SHRIMP_DEV Row16 load_row16(const unsigned char* src) {
  Row16 r;
  r.p0 = *reinterpret_cast<const u32x4*>(src);
  r.p1 = *reinterpret_cast<const u32x4*>(src + 16);
  return r;
}

SHRIMP_DEV float dot16(const Row16& a, const Row16& b) {
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned x = a.p0[w], y = b.p0[w];
    s = __builtin_amdgcn_fdot2(as_h2(x), as_h2(y), s, false);
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned x = a.p1[w], y = b.p1[w];
    s = __builtin_amdgcn_fdot2(as_h2(x), as_h2(y), s, false);
  }
  return s;
}

SHRIMP_DEV void fma_row16(float (&acc)[16], float p, const Row16& v) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned u = v.p0[w];
    const f16x2 h = as_h2(u);
    acc[2 * w] = fmaf(p, (float)h.x, acc[2 * w]);
    acc[2 * w + 1] = fmaf(p, (float)h.y, acc[2 * w + 1]);
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned u = v.p1[w];
    const f16x2 h = as_h2(u);
    acc[8 + 2 * w] = fmaf(p, (float)h.x, acc[8 + 2 * w]);
    acc[8 + 2 * w + 1] = fmaf(p, (float)h.y, acc[8 + 2 * w + 1]);
  }
}

// Workgroup: (position b, head pair p), 256 threads, D / 16 lanes per query row
// (each owning 16 of its D channels). LDS: the pair's 22 slot biases (fp32),
// then (STAGE) [K | V][head of pair][row][D] fp16. Rows are buffer accesses
// from the head pair's first head with 32-bit byte offsets (head h adds
// h times the head stride; the host checks that the strides are not negative
// and that a head pair's rows of a position span less than 2 GiB), so no
// access goes through a generic pointer chosen by the head index.
template <int D, bool STAGE>
__global__ __launch_bounds__(RA_THREADS) void ray_attn_kernel(const shrimp_ray_attn_args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  constexpr int LPR = D / 16;
  constexpr int RPP = RA_THREADS / LPR;
    const int npairs = (a.H + 1) >> 1;
  int b, p;
  if ((a.B & 7) == 0) {
    // Consecutive workgroups go to the eight XCDs in turn: keep the head pairs
    // of one position on one XCD (its L2 then holds the position's rows once).
    const int w = (int)blockIdx.x;
    const int kk = w >> 3;
    b = (kk / npairs) * 8 + (w & 7);
    p = kk % npairs;
  } else {
    b = (int)blockIdx.x / npairs;
    p = (int)blockIdx.x % npairs;
  }
  const int N = a.N;
  const int nh = min(2, a.H - 2 * p);
  SHRIMP_DCHECK(a.seq_lens[b] >= 0 && a.seq_lens[b] <= N, SHRIMP_DBG_SEQ_LEN);
  const int live_rows = min(max(a.seq_lens[b], 0), N);
  const int nst = STAGE ? live_rows : 0;
  const int part = (int)threadIdx.x % LPR;
  const bool axis = p < 3;

  // Per-head base pointers (the second head of an odd pair aliases the first
  // and is never used) and byte row strides.
  const unsigned char* qb[2];
  const unsigned char* kb[2];
  const unsigned char* vb[2];
  unsigned char* ob[2];
#pragma unroll
  for (int hl = 0; hl < 2; ++hl) {
    const int64_t hh = 2 * p + min(hl, nh - 1);
    qb[hl] = reinterpret_cast<const unsigned char*>(a.q + (int64_t)b * a.q_sb + hh * a.q_sh);
    kb[hl] = reinterpret_cast<const unsigned char*>(a.k + (int64_t)b * a.k_sb + hh * a.k_sh);
    vb[hl] = reinterpret_cast<const unsigned char*>(a.v + (int64_t)b * a.v_sb + hh * a.v_sh);
    ob[hl] = reinterpret_cast<unsigned char*>(a.out + (int64_t)b * a.o_sb + hh * a.o_sh);
  }
  const uint32_t qsn = (uint32_t)a.q_sn * 2, ksn = (uint32_t)a.k_sn * 2;
  const uint32_t vsn = (uint32_t)a.v_sn * 2, osn = (uint32_t)a.o_sn * 2;

  // slot biases of the pair: [hl][i], i = 0 self, 1 + t the axis slots
  float* sbias = reinterpret_cast<float*>(lds);
  if (threadIdx.x < 22) {
    const int hl = (int)threadIdx.x / 11, i = (int)threadIdx.x % 11;
    const int slot = i == 0 ? 0 : 1 + 10 * (axis ? p : 0) + (i - 1);
    const int hh = 2 * p + min(hl, nh - 1);
    sbias[threadIdx.x] = (float)__builtin_bit_cast(_Float16, a.slot_bias[slot * a.H + hh]);
  }
  const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qb[0], 0x7FFFFFFFu);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb[0], 0x7FFFFFFFu);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vb[0], 0x7FFFFFFFu);
  const __amdgpu_buffer_rsrc_t ors = make_rsrc(ob[0], 0x7FFFFFFFu);
  const uint32_t qhs = (uint32_t)(qb[1] - qb[0]), khs = (uint32_t)(kb[1] - kb[0]);
  const uint32_t vhs = (uint32_t)(vb[1] - vb[0]), ohs = (uint32_t)(ob[1] - ob[0]);
  unsigned char* rows = lds + RA_BIAS_LDS;
  if constexpr (STAGE) {
    constexpr int CPR = D / 8;  // 16-byte chunks per row and head
    const int per = nst * CPR;
#pragma unroll
    for (int tsr = 0; tsr < 2; ++tsr)
      for (int hl = 0; hl < nh; ++hl) {
        const uint32_t base = (uint32_t)hl * (tsr ? vhs : khs);
        const uint32_t sn = tsr ? vsn : ksn;
        unsigned char* dst = rows + (size_t)(tsr * 2 + hl) * N * D * 2;
        for (int c = (int)threadIdx.x; c < per; c += RA_THREADS) {
          const int j = c / CPR, ch = c % CPR;
          *reinterpret_cast<u32x4*>(dst + (uint32_t)(j * D + ch * 8) * 2) =
              buf_load16(tsr ? vrs : krs, base + (uint32_t)j * sn + ch * 16);
        }
      }
  }
  __syncthreads();

  // Key row fetch: the lane's 16 channels of row j of head (2p + hl). Rows
  // not staged in LDS are buffer loads from the head pair's base (a distinct
  // load kind, so the two paths never merge into one generic-pointer load).
  auto fetch = [&](int tsr, int hl, int j) -> Row16 {
    if (STAGE && j < nst)
      return load_row16(rows + (((size_t)(tsr * 2 + hl) * N + j) * D + part * 16) * 2);
    const uint32_t off = (uint32_t)hl * (tsr ? vhs : khs) + (uint32_t)j * (tsr ? vsn : ksn) + part * 32;
    Row16 r;
    r.p0 = buf_load16(tsr ? vrs : krs, off);
    r.p1 = buf_load16(tsr ? vrs : krs, off + 16);
    return r;
  };

  for (int r = (int)threadIdx.x / LPR; r < N; r += RPP) {
    if (r >= live_rows) {
      for (int hl = 0; hl < nh; ++hl) {
        const uint32_t off = (uint32_t)hl * ohs + (uint32_t)r * osn + part * 32;
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, ors, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, ors, off + 16, 0, 0);
      }
      continue;
    }
    const int32_t* ir = a.idx + (int64_t)b * a.idx_sb + (int64_t)r * a.idx_sn;
    int js[11];
    js[0] = ir[0];
#pragma unroll
    for (int t = 0; t < 10; ++t) js[1 + t] = axis ? ir[1 + 10 * p + t] : -1;
#pragma unroll
    for (int t = 0; t < 11; ++t) SHRIMP_DCHECK(js[t] >= -1, SHRIMP_DBG_RAY_INDEX);
    uint32_t rl4 = 0x05050505u;  // reach (own dir 0, own dir 1, opp dir 0, opp dir 1)
    if (a.blockers && axis) {
      const uint8_t* rl = a.raylen + (int64_t)b * a.rl_sb + (int64_t)r * a.rl_sn + 2 * p;
      rl4 = (uint32_t)rl[0] | ((uint32_t)rl[1] << 8) | ((uint32_t)rl[6] << 16) | ((uint32_t)rl[7] << 24);
    }

    for (int hl = 0; hl < nh; ++hl) {
      const int reach0 = (int)((rl4 >> (16 * hl)) & 0xFF);
      const int reach1 = (int)((rl4 >> (16 * hl + 8)) & 0xFF);
      // live slots as a per-lane bit mask (lane masks per slot would pin 22
      // scalar registers across the slot loops)
      uint32_t live = (unsigned)js[0] < (unsigned)N ? 1u : 0u;
#pragma unroll
      for (int t = 0; t < 10; ++t)
        live |= ((unsigned)js[1 + t] < (unsigned)N && (t % 5 + 1) <= (t < 5 ? reach0 : reach1) ? 1u : 0u)
                << (1 + t);

      Row16 q;
      {
        const uint32_t off = (uint32_t)hl * qhs + (uint32_t)r * qsn + part * 32;
        q.p0 = buf_load16(qrs, off);
        q.p1 = buf_load16(qrs, off + 16);
      }
      float s[11];
      float m = -INFINITY;
#pragma unroll
      for (int i = 0; i < 11; ++i) {
        s[i] = -INFINITY;
        if (live & (1u << i)) {
          float d = dot16(q, fetch(0, hl, js[i]));
#pragma unroll
          for (int x = 1; x < LPR; x <<= 1) d += __shfl_xor(d, x, 64);
          s[i] = d * inv_sqrt_d<D>() + sbias[hl * 11 + i];
          m = fmaxf(m, s[i]);
        }
      }
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
      float l = 0.f;
#pragma unroll
      for (int i = 0; i < 11; ++i) {
        if (live & (1u << i)) {
          const float pr = __builtin_amdgcn_exp2f((s[i] - m) * LOG2E_F);
          l += pr;
          fma_row16(acc, pr, fetch(1, hl, js[i]));
        }
      }
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      u32x4 o0, o1;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        o0[w] = pack_f16x2(acc[2 * w] * inv, acc[2 * w + 1] * inv);
        o1[w] = pack_f16x2(acc[8 + 2 * w] * inv, acc[8 + 2 * w + 1] * inv);
      }
      const uint32_t off = (uint32_t)hl * ohs + (uint32_t)r * osn + part * 32;
      __builtin_amdgcn_raw_buffer_store_b128(o0, ors, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(o1, ors, off + 16, 0, 0);
    }
  }
}

// ---- ray-tap conv + LayerNorm (K1) -------------------------------------------------

constexpr int RT_MB = 4;  // 16-row blocks per wave (64 rows)
constexpr int RT_MAX_N = 512;
constexpr int RT_MAX_WAVES = RT_MAX_N / (16 * RT_MB);

// Slot of step k = 1 for direction tap t = 1..6 (DIRECTIONS (1,0) (0,1) (-1,1)
// (-1,0) (0,-1) (1,-1) against the axes Q (1,0), R (0,1), QR (1,-1)):
// 1 + axis * 10 + dir * 5; step k adds k - 1.
__constant__ int RT_SLOT_BASE[6] = {1, 11, 26, 6, 16, 21};

__host__ __device__ constexpr int rt_row_stride(int cin) { return cin * 2 + 16; }
__host__ __device__ constexpr int rt_out_stride(int cout) { return cout * 2 + 16; }
// Bytes of the row region: the x rows (N + 1 of them) during the taps, the
// output rows (64 per wave) in the epilogue.
__host__ __device__ inline uint32_t rt_rows_bytes(int N, int cin, int cout, int waves) {
  const uint32_t xr = (uint32_t)(N + 1) * rt_row_stride(cin);
  const uint32_t orr = (uint32_t)waves * 64 * rt_out_stride(cout);
  return xr > orr ? xr : orr;
}

template <int CIN, int COUT>
constexpr uint32_t rt_wpack_bytes() {
  return (uint32_t)7 * CIN * COUT * 2;
}

// Packed weight fragment (step s = tap * KC + kc, output block nb): lane
// (lr, lg) holds W[tap][32 kc + 8 lg + e][16 nb + lr], e = 0..7, at byte
// ((s * NB + nb) * 64 + lane) * 16.
__global__ void raytap_pack_kernel(const uint16_t* __restrict__ w, int C, int Cout,
                                   uint16_t* __restrict__ out) {
  const int KC = C / 32, NB = Cout / 16;
  const int total = 7 * KC * NB * 64;
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= total) return;
  const int lane = i & 63, frag = i >> 6;
  const int nb = frag % NB, s = frag / NB;
  const int tap = s / KC, kc = s % KC;
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    out[(size_t)i * 8 + e] = w[((size_t)tap * C + kc * 32 + lg * 8 + e) * Cout + nb * 16 + lr];
}

SHRIMP_DEV f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int CIN, int COUT>
__global__ __launch_bounds__(64 * RT_MAX_WAVES) void conv_ln_raytap_kernel(
    const shrimp_raytap_args a) {
  constexpr int KC = CIN / 32, NB = COUT / 16, MB = RT_MB;
  constexpr int RS = rt_row_stride(CIN);
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int N = a.N;
  const int b = (int)blockIdx.x;
  const int lane = (int)threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  unsigned char* xs = lds;  // (N + 1) rows of RS bytes, later the output rows
  unsigned char* al = lds + rt_rows_bytes(N, CIN, COUT, (int)(blockDim.x >> 6));  // alpha (5, CIN) fp16

  // Stage the position's rows, the zero row N and alpha.
  {
    constexpr int CH = CIN / 8;
    const unsigned char* xb = reinterpret_cast<const unsigned char*>(a.x) + (int64_t)b * a.x_sb * 2;
    for (int c = (int)threadIdx.x; c < (N + 1) * CH; c += (int)blockDim.x) {
      const int j = c / CH, ch = c % CH;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (j < N) v = *reinterpret_cast<const u32x4*>(xb + (int64_t)j * a.x_sn * 2 + ch * 16);
      *reinterpret_cast<u32x4*>(xs + j * RS + ch * 16) = v;
    }
    for (int c = (int)threadIdx.x; c < RAY_STEPS * CH; c += (int)blockDim.x)
      *reinterpret_cast<u32x4*>(al + c * 16) =
          *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned char*>(a.alpha) + c * 16);
  }

  // This lane's rows: wave * 64 + mb * 16 + lr.
  int rn[MB];
  bool rv[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    rn[mb] = wave * 64 + mb * 16 + lr;
    rv[mb] = rn[mb] < N;
  }
  const int32_t* rib = a.ray_idx + (int64_t)b * a.r_sb;
  const uint8_t* reb = a.reach + (int64_t)b * a.re_sb;

  f32x4 acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const f32x4 bb = *reinterpret_cast<const f32x4*>(a.bias + nb * 16 + lg * 4);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = bb;
  }
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.packed_w, rt_wpack_bytes<CIN, COUT>());
  auto wload = [&](int s, u32x4 (&w)[NB]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) w[nb] = buf_load16(wr, (uint32_t)(((s * NB + nb) * 64 + lane) * 16));
  };

  // Centre rows (tap 0): LDS row index, N for absent.
  uint32_t crow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int j = rv[mb] ? a.gather_idx[(int64_t)b * a.g_sb + (int64_t)rn[mb] * a.g_sn] : N;
    SHRIMP_DCHECK(j >= -1, SHRIMP_DBG_RAY_INDEX);
    crow[mb] = (unsigned)j < (unsigned)N ? (uint32_t)j : (uint32_t)N;
  }
  // Side of the lane's two 4-channel halves of chunk kc, (c % corb) >= corb / 2:
  // bit 2 kc + h set for the opp side.
  uint32_t sidebits = 0;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = kc * 32 + lg * 8 + h * 4;
      if ((c % a.corb) >= (a.corb >> 1)) sidebits |= 1u << (2 * kc + h);
    }

  // Ray rows and reach of one direction tap for row wave * 64 + lane, loaded
  // one tap ahead so the global latency hides behind the previous tap.
  const int trow = wave * 64 + lane;
  int pj[RAY_STEPS];
  uint32_t preach = 0;
  auto tap_fetch = [&](int t) {
#pragma unroll
    for (int k = 0; k < RAY_STEPS; ++k) pj[k] = N;
    preach = 0;
    if (trow < N) {
      const int32_t* ir = rib + (int64_t)trow * a.r_sn + RT_SLOT_BASE[t];
#pragma unroll
      for (int k = 0; k < RAY_STEPS; ++k) {
        pj[k] = ir[k];
        SHRIMP_DCHECK(pj[k] >= -1, SHRIMP_DBG_RAY_INDEX);
      }
      const uint8_t* re = reb + (int64_t)trow * a.re_sn;
      preach = (uint32_t)re[t] | ((uint32_t)re[6 + t] << 8);
    }
  };
  tap_fetch(0);

  __syncthreads();

  // Tap 0: two weight buffers (nothing else is live here); the last chunk
  // requests the first step of tap 1.
  u32x4 w[NB];
  {
    u32x4 wa[NB], wb[NB];
    wload(0, wa);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      u32x4 (&wc)[NB] = (kc & 1) ? wb : wa;
      u32x4 (&wn)[NB] = (kc & 1) ? wa : wb;
      wload(kc + 1, wn);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const u32x4 xf = *reinterpret_cast<const u32x4*>(xs + crow[mb] * RS + (kc * 32 + lg * 8) * 2);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma_f16(wc[nb], xf, acc[nb][mb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    u32x4 (&wl)[NB] = (KC & 1) ? wb : wa;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) w[nb] = wl[nb];
  }

  // Taps 1..6. Per tap, lane l of each wave writes, for row wave * 64 + l, the
  // visible row of every step and side into the wave's slice of `vt` (5 dwords,
  // own | opp << 16, N = the zero row; 8 dwords per row); every chunk of the tap
  // reads it back for its rows. The slice belongs to one wave and a wave's LDS
  // accesses complete in issue order, so no workgroup barrier is needed.
  uint32_t* vt = reinterpret_cast<uint32_t*>(al + RAY_STEPS * CIN * 2) + wave * 64 * 8;
  for (int t = 0; t < 6; ++t) {
    {
      const int r0 = (int)(preach & 0xFF), r1 = (int)(preach >> 8);
      uint32_t vr[RAY_STEPS];
#pragma unroll
      for (int k = 0; k < RAY_STEPS; ++k) {
        const bool pres = (unsigned)pj[k] < (unsigned)N;
        const uint32_t own = pres && k + 1 <= r0 ? (uint32_t)pj[k] : (uint32_t)N;
        const uint32_t opp = pres && k + 1 <= r1 ? (uint32_t)pj[k] : (uint32_t)N;
        vr[k] = own | (opp << 16);
      }
      *reinterpret_cast<u32x4*>(vt + lane * 8) = u32x4{vr[0], vr[1], vr[2], vr[3]};
      vt[lane * 8 + 4] = vr[4];
    }
    if (t + 1 < 6) tap_fetch(t + 1);
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    // Table entries of the next row block, read one block ahead (they do not
    // depend on the chunk, so the block after the last is block 0 again).
    auto vt_read = [&](int mb, uint32_t (&v)[RAY_STEPS]) {
      const uint32_t* vp = vt + (mb * 16 + lr) * 8;
      const u32x4 v4 = *reinterpret_cast<const u32x4*>(vp);
      v[0] = v4[0];
      v[1] = v4[1];
      v[2] = v4[2];
      v[3] = v4[3];
      v[4] = vp[4];
    };
    uint32_t vnext[RAY_STEPS];
    vt_read(0, vnext);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      // alpha of the lane's 8 channels, steps 1..5
      u32x4 av[RAY_STEPS];
#pragma unroll
      for (int k = 0; k < RAY_STEPS; ++k)
        av[k] = *reinterpret_cast<const u32x4*>(al + (k * CIN + kc * 32 + lg * 8) * 2);
      const int sh0 = ((sidebits >> (2 * kc)) & 1u) * 16, sh1 = ((sidebits >> (2 * kc + 1)) & 1u) * 16;
      const uint32_t cb = (uint32_t)(kc * 32 + lg * 8) * 2;
      const int next = (1 + t) * KC + kc + 1;  // weight step after this one
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        u32x2 xr[RAY_STEPS][2];
#pragma unroll
        for (int k = 0; k < RAY_STEPS; ++k) {
          const uint32_t j0 = (vnext[k] >> sh0) & 0xFFFFu;
          const uint32_t j1 = (vnext[k] >> sh1) & 0xFFFFu;
          xr[k][0] = *reinterpret_cast<const u32x2*>(xs + j0 * RS + cb);
          xr[k][1] = *reinterpret_cast<const u32x2*>(xs + j1 * RS + cb + 8);
        }
        vt_read(mb + 1 < MB ? mb + 1 : 0, vnext);
        float sum[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) sum[e] = 0.f;
#pragma unroll
        for (int k = 0; k < RAY_STEPS; ++k) {
          const unsigned xw[4] = {xr[k][0][0], xr[k][0][1], xr[k][1][0], xr[k][1][1]};
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) {
            const unsigned au = av[k][w2];
            const f16x2 ah = as_h2(au), xh = as_h2(xw[w2]);
            sum[2 * w2] = fmaf((float)ah.x, (float)xh.x, sum[2 * w2]);
            sum[2 * w2 + 1] = fmaf((float)ah.y, (float)xh.y, sum[2 * w2 + 1]);
          }
        }
        u32x4 bf;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) bf[w2] = pack_f16x2(sum[2 * w2], sum[2 * w2 + 1]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb][mb] = mfma_f16(w[nb], bf, acc[nb][mb]);
        // The last block's products hold the step's weights; the next step's
        // fragments load into the same registers right behind them.
        if (mb == MB - 1 && next < 7 * KC) wload(next, w);
        // Keep the next row block's loads behind this block's products (hoisting all
        // four blocks' loads overflows the register budget).
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // LayerNorm over COUT (lane: channels 16 nb + 4 lg + j of row rn[mb]), ReLU, mask:
  // the statistics of all row blocks first, then the output block by block, so
  // only one block's LayerNorm parameters are live next to the accumulators.
  const uint8_t* mk = a.mask + (int64_t)b * N;
  float mean[MB], rstd[MB];
  bool live[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float s = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) s += acc[nb][mb][j];
    mean[mb] = sum_groups_swap(s) * (1.0f / COUT);
    float q = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float c = acc[nb][mb][j] - mean[mb];
        q = fmaf(c, c, q);
      }
    rstd[mb] = rsqrtf(sum_groups_swap(q) * (1.0f / COUT) + a.eps);
    live[mb] = rv[mb] && mk[rn[mb]] != 0;
  }
  // The output rows go through LDS (each wave's 64 rows in its own slice over
  // the x rows, which every wave has finished reading) and leave as whole
  // 16-byte row pieces: 8-byte stores per lane would write 32-byte segments.
  __syncthreads();
  constexpr int OS = rt_out_stride(COUT);
  unsigned char* ob = xs + (size_t)wave * 64 * OS;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int c0 = nb * 16 + lg * 4;
    const f32x4 lw = *reinterpret_cast<const f32x4*>(a.ln_w + c0);
    const f32x4 lb = *reinterpret_cast<const f32x4*>(a.ln_b + c0);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float y[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = (acc[nb][mb][j] - mean[mb]) * rstd[mb] * lw[j] + lb[j];
        if (a.relu) v = fmaxf(v, 0.f);
        y[j] = live[mb] ? v : 0.f;
      }
      *reinterpret_cast<u32x2*>(ob + (mb * 16 + lr) * OS + c0 * 2) =
          u32x2{pack_f16x2(y[0], y[1]), pack_f16x2(y[2], y[3])};
    }
  }
  // The slice belongs to this wave and its LDS accesses complete in issue order.
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  constexpr int CPR = COUT / 8;  // 16-byte pieces per output row
  const int ch = lane & 15;
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int r = it * 4 + (lane >> 4);
    const int row = wave * 64 + r;
    if (ch < CPR && row < N) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(ob + r * OS + ch * 16);
      *reinterpret_cast<u32x4*>(a.out + (int64_t)b * a.o_sb + (int64_t)row * a.o_sn + ch * 8) = v;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int D>
int launch_ray_attn(const shrimp_ray_attn_args& a, bool stage, hipStream_t st) {
  const int npairs = (a.H + 1) / 2;
  const dim3 grid((unsigned)((int64_t)a.B * npairs));
  if (stage) {
    const uint32_t lds = RA_BIAS_LDS + 8u * (uint32_t)a.N * D;
    hipLaunchKernelGGL((ray_attn_kernel<D, true>), grid, dim3(RA_THREADS), lds, st, a);
  } else {
    hipLaunchKernelGGL((ray_attn_kernel<D, false>), grid, dim3(RA_THREADS), RA_BIAS_LDS, st, a);
  }
  return check_launch("ray_attn");
}

template <int CIN>
int launch_raytap_cin(const shrimp_raytap_args& a, size_t lds, hipStream_t st) {
  const int waves = (a.N + 16 * RT_MB - 1) / (16 * RT_MB);
  const dim3 grid((unsigned)a.B), block((unsigned)(64 * waves));
  switch (a.Cout) {
    case 64: hipLaunchKernelGGL((conv_ln_raytap_kernel<CIN, 64>), grid, block, lds, st, a); break;
    case 96: hipLaunchKernelGGL((conv_ln_raytap_kernel<CIN, 96>), grid, block, lds, st, a); break;
    default: hipLaunchKernelGGL((conv_ln_raytap_kernel<CIN, 128>), grid, block, lds, st, a); break;
  }
  return check_launch("conv_ln_raytap");
}

bool raytap_shape_ok(int C, int Cout) {
  return (C == 64 || C == 96 || C == 128) && (Cout == 64 || Cout == 96 || Cout == 128);
}

}  // namespace

extern "C" int shrimp_ray_attn_variant(int v) {
  if (v != 0 && v != 1) return g_ray_variant.load();
  return g_ray_variant.exchange(v);
}

extern "C" int shrimp_ray_attn(const shrimp_ray_attn_args* a, void* stream) {
  SHRIMP_REQUIRE(a, "ray_attn: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->H >= 1 && a->H <= kMaxDim && a->N >= 1 && a->N <= kMaxDim, "ray_attn: bad shape B=%d H=%d N=%d", a->B,
                 a->H, a->N);
  SHRIMP_REQUIRE(a->D == 16 || a->D == 32 || a->D == 64 || a->D == 128,
                 "ray_attn: head dim %d not in {16, 32, 64, 128}", a->D);
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->q && a->k && a->v && a->out && a->idx && a->slot_bias && a->seq_lens,
                 "ray_attn: null pointer");
  SHRIMP_REQUIRE(!a->blockers || a->raylen, "ray_attn: blockers need raylen");
  SHRIMP_REQUIRE(aligned16(a->q) && aligned16(a->k) && aligned16(a->v) && aligned16(a->out),
                 "ray_attn: q/k/v/out must be 16-byte aligned");
  const int64_t st[12] = {a->q_sb, a->q_sh, a->q_sn, a->k_sb, a->k_sh, a->k_sn,
                          a->v_sb, a->v_sh, a->v_sn, a->o_sb, a->o_sh, a->o_sn};
  for (int i = 0; i < 12; ++i)
    SHRIMP_REQUIRE(st[i] % 8 == 0 && st[i] >= 0 && st[i] < (1LL << 31),
                   "ray_attn: q/k/v/out strides must be multiples of 8 elements in [0, 2^31)");
  SHRIMP_REQUIRE(strides_ok({a->idx_sb, a->idx_sn, a->rl_sb, a->rl_sn}),
                 "ray_attn: idx / raylen strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->idx_sn >= RAY_SLOT_COUNT && a->idx_sb >= (int64_t)a->N * a->idx_sn - a->idx_sn + RAY_SLOT_COUNT,
                 "ray_attn: idx rows must hold 32 slots");
  SHRIMP_REQUIRE(!a->blockers || a->rl_sn >= 12, "ray_attn: raylen rows must hold 12 slots");
  const int64_t rsn[4] = {a->q_sn, a->k_sn, a->v_sn, a->o_sn};
  const int64_t rsh[4] = {a->q_sh, a->k_sh, a->v_sh, a->o_sh};
  for (int i = 0; i < 4; ++i)
    SHRIMP_REQUIRE(rsn[i] >= a->D && ((int64_t)a->N * rsn[i] + rsh[i]) * 2 < (1LL << 31),
                   "ray_attn: a head pair's rows of a position must span less than 2 GiB");
  SHRIMP_REQUIRE((int64_t)a->B * ((a->H + 1) / 2) < (1LL << 31), "ray_attn: grid too large");
  const bool stage = g_ray_variant == 0 && 8u * (uint64_t)a->N * a->D <= RA_STAGE_MAX_LDS;
  hipStream_t s = as_stream(stream);
  switch (a->D) {
    case 16: return launch_ray_attn<16>(*a, stage, s);
    case 32: return launch_ray_attn<32>(*a, stage, s);
    case 64: return launch_ray_attn<64>(*a, stage, s);
    default: return launch_ray_attn<128>(*a, stage, s);
  }
}

extern "C" size_t shrimp_raytap_wpack_bytes(int C, int Cout) {
  return raytap_shape_ok(C, Cout) ? (size_t)7 * C * Cout * 2 : 0;
}

extern "C" int shrimp_pack_raytap_weight(const uint16_t* w, int C, int Cout, void* packed,
                                         void* stream) {
  SHRIMP_REQUIRE(raytap_shape_ok(C, Cout), "pack_raytap_weight: C=%d Cout=%d not in {64, 96, 128}",
                 C, Cout);
  SHRIMP_REQUIRE(w && packed, "pack_raytap_weight: null pointer");
  const int total = 7 * (C / 32) * (Cout / 16) * 64;
  hipLaunchKernelGGL(raytap_pack_kernel, dim3((total + 255) / 256), dim3(256), 0,
                     as_stream(stream), w, C, Cout, reinterpret_cast<uint16_t*>(packed));
  return check_launch("pack_raytap_weight");
}

extern "C" int shrimp_conv_ln_raytap(const shrimp_raytap_args* a, void* stream) {
  SHRIMP_REQUIRE(a, "conv_ln_raytap: null args");
  SHRIMP_REQUIRE(raytap_shape_ok(a->C, a->Cout), "conv_ln_raytap: C=%d Cout=%d not in {64, 96, 128}",
                 a->C, a->Cout);
  SHRIMP_REQUIRE(a->B >= 0 && a->N >= 1 && a->N <= RT_MAX_N, "conv_ln_raytap: N=%d not in [1, %d]",
                 a->N, RT_MAX_N);
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->x && a->gather_idx && a->mask && a->packed_w && a->bias && a->ln_w && a->ln_b &&
                     a->ray_idx && a->reach && a->alpha && a->out,
                 "conv_ln_raytap: null pointer");
  SHRIMP_REQUIRE(strides_ok({a->x_sb, a->x_sn, a->o_sb, a->o_sn, a->g_sb, a->g_sn, a->r_sb, a->r_sn,
                             a->re_sb, a->re_sn}),
                 "conv_ln_raytap: strides outside [0, 2^31)");
  SHRIMP_REQUIRE(a->corb >= 8 && a->corb % 8 == 0 && a->C % a->corb == 0,
                 "conv_ln_raytap: corb=%d must divide C=%d and be a multiple of 8", a->corb, a->C);
  SHRIMP_REQUIRE(aligned16(a->x) && a->x_sb % 8 == 0 && a->x_sn % 8 == 0 && a->x_sn >= a->C,
                 "conv_ln_raytap: x must be 16-byte aligned with strides multiples of 8");
  SHRIMP_REQUIRE(aligned16(a->out) && a->o_sb % 8 == 0 && a->o_sn % 8 == 0 && a->o_sn >= a->Cout,
                 "conv_ln_raytap: out must be 16-byte aligned with strides multiples of 8");
  SHRIMP_REQUIRE(aligned16(a->alpha) && aligned16(a->bias) && aligned16(a->ln_w) &&
                     aligned16(a->ln_b) && aligned16(a->packed_w),
                 "conv_ln_raytap: alpha / bias / ln params / weights must be 16-byte aligned");
  SHRIMP_REQUIRE(a->r_sn >= RAY_SLOT_COUNT && a->re_sn >= 12 && a->g_sn >= 1,
                 "conv_ln_raytap: ray_idx rows need 32 slots, reach rows 12 bytes");
  const int waves = (a->N + 16 * RT_MB - 1) / (16 * RT_MB);
  const size_t lds = (size_t)rt_rows_bytes(a->N, a->C, a->Cout, waves) +
                     (size_t)RAY_STEPS * a->C * 2 + (size_t)waves * 64 * 8 * 4;
  SHRIMP_REQUIRE(lds <= (size_t)max_lds_per_block(), "conv_ln_raytap: needs %zu bytes of LDS", lds);
  hipStream_t s = as_stream(stream);
  switch (a->C) {
    case 64: return launch_raytap_cin<64>(*a, lds, s);
    case 96: return launch_raytap_cin<96>(*a, lds, s);
    default: return launch_raytap_cin<128>(*a, lds, s);
  }
}
