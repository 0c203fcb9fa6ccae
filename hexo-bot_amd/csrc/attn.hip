// Fused relative-position-biased, key-masked attention for gfx950.
//
// Semantics: RelPosAttention's softmax(q k^T / sqrt(d) + bias) v with the
// per-block bias table (packages/shrimp/python/shrimp/model.py:448-492,
// 677-760) and the serve kernel's key bound (_triton_attn.py:59-130):
// keys >= seq_lens[b] are never visited, pad keys inside it get weight 0.
//
// One workgroup = one position x HG heads; K (key-major) and V (transposed,
// dim-major) of those heads, the per-key coordinates and the heads' bias
// columns are staged in LDS once, then each wave walks 16-query blocks.
// Everything is kept in the "transposed" MFMA orientation so no value ever
// changes lanes:
//   S^T = K Q^T  (v_mfma_f32_16x16x16_bf16): lane l holds keys 4*(l/16)+j of
//                query l%16 — exactly the B operand layout of P^T below;
//   O^T += V^T P^T: lane l holds dims 4*(l/16)+j of query l%16, so the online
//                softmax rescale uses the lane's own running max.
// The bias row of a cell pair is computed in-kernel from coordinates through
// the clamped offset LUT (coords mode) or read from the reference's uint8
// pair tensor (pair mode); the pair index is computed once and reused by the
// HG heads. Softmax runs in base 2 with log2(e) folded into the scale and the
// staged bias table; statistics are fp32.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

#define SHRIMP_LOG2E 1.4426950408889634f
#define SHRIMP_NEG_BIG (-1.0e30f)

enum : int { KEY_CELL = 0, KEY_TOKEN = 1, KEY_DEAD = 2 };

// Max over the 4 lane groups (l / 16) that share l % 16, on VALU lane swaps.
SHRIMP_DEV float max_groups_swap(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

struct AttnLds {
  unsigned short* Ks;  // [HG][SP][DP] key-major
  unsigned short* Vt;  // [HG][DP][SP] dim-major
  int2* kqr;           // [SP] key coordinates
  int* kcls;           // [SP] KEY_CELL / KEY_TOKEN / KEY_DEAD
  int* blk_gen;        // [SP / 16] 1 if the 16-key block holds a token or dead key
  float* tab;          // [npos][HG] bias columns, log2(e) folded
};

struct AttnQuery {
  int query, qq, qr;
  bool qtok, qv;
};

// One chunk of NBK 16-key blocks for all HG heads of one 16-query block.
// GENERAL handles token rows/columns, dead keys and the key bound; the fast
// path assumes every key of the chunk is a live cell and the query is a cell.
template <int DP, int HG, bool PAIR, int NBK, bool GENERAL>
SHRIMP_DEV void attn_chunk(const shrimp_attn_args& a, const AttnLds& s, const AttnQuery& qi,
                           int kb0, int L, int SP, int lr, int lg, float qk_scale, int npos,
                           const u32x2 (&qf)[HG][DP / 16], float (&m)[HG], float (&l)[HG],
                           f32x4 (&o)[HG][DP / 16]) {
  constexpr int KD = DP / 16;
  const int M = a.lut_m;
  const int W = 2 * M + 1;
  f32x4 sc4[HG][NBK];
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const u32x2 kf = *reinterpret_cast<const u32x2*>(
            s.Ks + (h * SP + (kb0 + kb) * 16 + lr) * DP + kd * 16 + lg * 4);
        acc = mfma16x16x16(kf, qf[h][kd], acc);
      }
      sc4[h][kb] = acc;
    }
  int pos[NBK][4];
  bool live[NBK][4];
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = (kb0 + kb) * 16 + lg * 4 + j;
      live[kb][j] = true;
      if (PAIR) {
        if (GENERAL) live[kb][j] = key < L;
        const uint8_t* prow = a.pair + (int64_t)blockIdx.y * a.p_sb + (int64_t)qi.query * a.p_sq;
        const int p = (live[kb][j] && qi.qv) ? (int)prow[key] : 0;
        pos[kb][j] = p < npos ? p : npos - 1;
      } else {
        const int2 kk = s.kqr[key];
        const int dq = min(max(kk.x - qi.qq, -M), M);
        const int dr = min(max(kk.y - qi.qr, -M), M);
        int p = (dq + M) * W + (dr + M);
        if (GENERAL) {
          const int cls = s.kcls[key];
          live[kb][j] = cls != KEY_DEAD;
          const int tp = qi.qtok ? W * W + 2 : W * W;  // key token: (token q | cell q)
          const int cp = qi.qtok ? W * W + 1 : p;      // key cell
          p = cls == KEY_TOKEN ? tp : cp;
        }
        pos[kb][j] = p;
      }
    }
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    float sc[NBK][4];
    float mx = SHRIMP_NEG_BIG;
#pragma unroll
    for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = sc4[h][kb][j] * qk_scale + s.tab[pos[kb][j] * HG + h];
        if (GENERAL) v = live[kb][j] ? v : SHRIMP_NEG_BIG;
        sc[kb][j] = v;
        mx = fmaxf(mx, v);
      }
    mx = max_groups_swap(mx);
    const float mnew = fmaxf(m[h], mx);
    const float alpha = __builtin_amdgcn_exp2f(m[h] - mnew);
    m[h] = mnew;
    float ps = 0.f;
    u32x2 pf[NBK];
#pragma unroll
    for (int kb = 0; kb < NBK; ++kb) {
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[j] = __builtin_amdgcn_exp2f(sc[kb][j] - mnew);
        if (GENERAL) p[j] = live[kb][j] ? p[j] : 0.f;
        ps += p[j];
      }
      pf[kb].x = pack_bf16x2(p[0], p[1]);
      pf[kb].y = pack_bf16x2(p[2], p[3]);
    }
    l[h] = l[h] * alpha + ps;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      f32x4 acc = o[h][kd] * alpha;
#pragma unroll
      for (int kb = 0; kb < NBK; ++kb) {
        const u32x2 vf = *reinterpret_cast<const u32x2*>(
            s.Vt + (h * DP + kd * 16 + lr) * SP + (kb0 + kb) * 16 + lg * 4);
        acc = mfma16x16x16(vf, pf[kb], acc);
      }
      o[h][kd] = acc;
    }
  }
}

template <int DP, int HG, bool PAIR>
__global__ __launch_bounds__(256) void attn_kernel(const shrimp_attn_args a, float qk_scale,
                                                   uint32_t qkv_bytes, int npos) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int KD = DP / 16;
  const int b = blockIdx.y;
  const int h0 = blockIdx.x * HG;
  const int S = a.S;
  const int SP = (S + 15) & ~15;
  int L = a.seq_lens[b];
  L = L < 0 ? 0 : (L > S ? S : L);
  const int LP = (L + 15) & ~15;
  const int nt = a.n_tokens;
  const int NC = S - nt;

  AttnLds s;
  s.Ks = reinterpret_cast<unsigned short*>(smem);
  s.Vt = s.Ks + HG * SP * DP;
  s.kqr = reinterpret_cast<int2*>(s.Vt + HG * DP * SP);
  s.kcls = reinterpret_cast<int*>(s.kqr + SP);
  s.blk_gen = s.kcls + SP;
  s.tab = reinterpret_cast<float*>(s.blk_gen + SP / 16);

  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q, qkv_bytes);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.k, qkv_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.v, qkv_bytes);
  const int64_t pos_base = (int64_t)b * a.qkv_sb;

  // ---- stage K (key-major) ---------------------------------------------------
  constexpr int CH = DP / 8;
  for (int i = tid; i < HG * LP * CH; i += 256) {
    const int h = i / (LP * CH);
    const int rem = i - h * LP * CH;
    const int key = rem / CH;
    const int ch = rem - key * CH;
    const uint32_t off =
        key < L ? (uint32_t)((pos_base + (int64_t)(h0 + h) * a.qkv_sh + key * DP + ch * 8) * 2)
                : SHRIMP_OOB_OFFSET;
    *reinterpret_cast<u32x4*>(s.Ks + (h * SP + key) * DP + ch * 8) = buf_load16(krs, off);
  }
  // ---- stage V^T (dim-major), keys (2k, 2k+1) packed per dword -------------------
  for (int i = tid; i < HG * (LP / 2) * CH; i += 256) {
    const int h = i / ((LP / 2) * CH);
    const int rem = i - h * (LP / 2) * CH;
    const int kp = rem / CH;
    const int ch = rem - kp * CH;
    const int key = 2 * kp;
    const int64_t e0 = pos_base + (int64_t)(h0 + h) * a.qkv_sh + key * DP + ch * 8;
    const u32x4 v0 = buf_load16(vrs, key < L ? (uint32_t)(e0 * 2) : SHRIMP_OOB_OFFSET);
    const u32x4 v1 = buf_load16(vrs, key + 1 < L ? (uint32_t)((e0 + DP) * 2) : SHRIMP_OOB_OFFSET);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int d = ch * 8 + 2 * w;
      unsigned* lo = reinterpret_cast<unsigned*>(s.Vt + (h * DP + d) * SP + key);
      unsigned* hi = reinterpret_cast<unsigned*>(s.Vt + (h * DP + d + 1) * SP + key);
      *lo = (v0[w] & 0xFFFFu) | (v1[w] << 16);
      *hi = (v0[w] >> 16) | (v1[w] & 0xFFFF0000u);
    }
  }
  // ---- key classes / coordinates / per-block flags ---------------------------------
  if (!PAIR) {
    for (int key = tid; key < LP; key += 256) {
      int q = 0, r = 0, cls = KEY_DEAD;
      if (key < nt) {
        cls = KEY_TOKEN;
      } else if (key < L) {
        const int64_t cell = (int64_t)b * NC + (key - nt);
        q = a.coords[cell * 2];
        r = a.coords[cell * 2 + 1];
        cls = a.mask[cell] ? KEY_CELL : KEY_DEAD;
      }
      s.kqr[key] = make_int2(q, r);
      s.kcls[key] = cls;
    }
  }
  for (int blk = tid; blk < LP / 16; blk += 256) {
    int gen = 0;
    for (int j = 0; j < 16; ++j) {
      const int key = blk * 16 + j;
      if (key >= L || key < nt) gen = 1;
      else if (!PAIR && !a.mask[(int64_t)b * NC + (key - nt)]) gen = 1;
    }
    s.blk_gen[blk] = gen;
  }
  // ---- bias columns of this head group --------------------------------------------
  for (int i = tid; i < npos * HG; i += 256) {
    const int pos = i / HG;
    const int h = i - pos * HG;
    s.tab[i] = PAIR ? a.table2[pos * a.H + h0 + h] * SHRIMP_LOG2E : a.btab[pos * a.H + h0 + h];
  }
  __syncthreads();

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int nkb = LP / 16;

  for (int qb = wave; qb * 16 < L; qb += 4) {
    AttnQuery qi;
    qi.query = qb * 16 + lr;
    qi.qv = qi.query < L;
    qi.qtok = qi.query < nt;
    qi.qq = 0;
    qi.qr = 0;
    if (!PAIR) {
      const int2 qc = s.kqr[qi.query];
      qi.qq = qc.x;
      qi.qr = qc.y;
    }
    const bool qgen = qb * 16 < nt;  // wave-uniform
    u32x2 qf[HG][KD];
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const int64_t e = pos_base + (int64_t)(h0 + h) * a.qkv_sh + qi.query * DP + kd * 16 + lg * 4;
        qf[h][kd] = buf_load8(qrs, qi.qv ? (uint32_t)(e * 2) : SHRIMP_OOB_OFFSET);
      }
    float m[HG], l[HG];
    f32x4 o[HG][KD];
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      m[h] = SHRIMP_NEG_BIG;
      l[h] = 0.f;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) o[h][kd] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    int kb = 0;
    while (kb < nkb) {
      if (nkb - kb >= 4) {
        const bool gen = qgen || (s.blk_gen[kb] | s.blk_gen[kb + 1] | s.blk_gen[kb + 2] |
                                  s.blk_gen[kb + 3]);
        if (gen)
          attn_chunk<DP, HG, PAIR, 4, true>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, qf, m, l, o);
        else
          attn_chunk<DP, HG, PAIR, 4, false>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, qf, m, l, o);
        kb += 4;
      } else {
        if (qgen || s.blk_gen[kb])
          attn_chunk<DP, HG, PAIR, 1, true>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, qf, m, l, o);
        else
          attn_chunk<DP, HG, PAIR, 1, false>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, qf, m, l, o);
        kb += 1;
      }
    }

#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float lt = sum_lane_groups(l[h]);
      const float inv = lt > 0.f ? 1.0f / lt : 0.f;
      if (!qi.qv) continue;
      unsigned short* orow = static_cast<unsigned short*>(a.o) + (int64_t)b * a.o_sb +
                             (int64_t)(h0 + h) * a.o_sh + (int64_t)qi.query * a.o_sr;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const int e = kd * 16 + lg * 4;
        if (e < a.d) {
          u32x2 pk;
          pk.x = pack_bf16x2(o[h][kd][0] * inv, o[h][kd][1] * inv);
          pk.y = pack_bf16x2(o[h][kd][2] * inv, o[h][kd][3] * inv);
          *reinterpret_cast<u32x2*>(orow + e) = pk;
        }
      }
    }
  }

  // Query rows past the live bound store zeros.
  const int dq4 = a.d / 4;
  for (int i = tid; i < (S - L) * HG * dq4; i += 256) {
    const int row = L + i / (HG * dq4);
    const int rem = i - (row - L) * HG * dq4;
    const int h = rem / dq4;
    const int e = (rem - h * dq4) * 4;
    unsigned short* orow = static_cast<unsigned short*>(a.o) + (int64_t)b * a.o_sb +
                           (int64_t)(h0 + h) * a.o_sh + (int64_t)row * a.o_sr;
    *reinterpret_cast<u32x2*>(orow + e) = u32x2{0u, 0u};
  }
}

static size_t attn_smem_bytes(int DP, int HG, int S, int npos) {
  const int SP = (S + 15) & ~15;
  return (size_t)2 * HG * SP * DP * 2 + (size_t)SP * (8 + 4) + (size_t)(SP / 16) * 4 +
         (size_t)npos * HG * 4;
}

template <int DP, int HG, bool PAIR>
static int launch_attn(const shrimp_attn_args* a, float qk_scale, uint32_t qkv_bytes, int npos,
                       hipStream_t st) {
  const size_t smem = attn_smem_bytes(DP, HG, a->S, npos);
  dim3 grid(a->H / HG, a->B);
  hipLaunchKernelGGL((attn_kernel<DP, HG, PAIR>), grid, dim3(256), smem, st, *a, qk_scale,
                     qkv_bytes, npos);
  return check_launch("attn");
}

// LDS budget per workgroup kept at 64 KiB so several groups share a CU.
static const size_t kAttnSmemCap = 64 * 1024;

template <bool PAIR>
static int dispatch_attn(const shrimp_attn_args* a, float qk_scale, uint32_t qkv_bytes, int npos,
                         hipStream_t st) {
#define SHRIMP_ATTN_DP(DPV)                                                          \
  if (a->dpad == DPV) {                                                              \
    if (a->H % 2 == 0 && attn_smem_bytes(DPV, 2, a->S, npos) <= kAttnSmemCap)        \
      return launch_attn<DPV, 2, PAIR>(a, qk_scale, qkv_bytes, npos, st);            \
    if (attn_smem_bytes(DPV, 1, a->S, npos) <= kAttnSmemCap)                          \
      return launch_attn<DPV, 1, PAIR>(a, qk_scale, qkv_bytes, npos, st);            \
    return set_error(SHRIMP_EINVAL, "attn: sequence %d too long for LDS staging", a->S); \
  }
  SHRIMP_ATTN_DP(16)
  SHRIMP_ATTN_DP(32)
  SHRIMP_ATTN_DP(64)
#undef SHRIMP_ATTN_DP
  return set_error(SHRIMP_EINVAL, "attn: unsupported padded head dim %d", a->dpad);
}

// btab[pos, h] = log2(e) * table[lut[pos], h]; three token rows appended.
__global__ void attn_bias_table_kernel(const float* __restrict__ table, int table_rows, int H,
                                       const uint8_t* __restrict__ lut, int npos_lut, int r_ct,
                                       int r_tc, int r_tt, float* __restrict__ btab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (npos_lut + 3) * H) return;
  const int pos = i / H;
  const int h = i - pos * H;
  int row;
  if (pos < npos_lut) row = lut[pos];
  else row = pos == npos_lut ? r_ct : (pos == npos_lut + 1 ? r_tc : r_tt);
  row = row < table_rows ? row : table_rows - 1;
  btab[i] = table[row * H + h] * SHRIMP_LOG2E;
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_attn_bias_table(const float* table, int table_rows, int H,
                                      const uint8_t* lut, int lut_m, int tok_row_ct,
                                      int tok_row_tc, int tok_row_tt, float* btab, void* stream) {
  SHRIMP_REQUIRE(table && lut && btab, "attn_bias_table: null pointer");
  SHRIMP_REQUIRE(table_rows > 0 && H > 0 && lut_m >= 0, "attn_bias_table: bad sizes");
  const int w = 2 * lut_m + 1;
  const int total = (w * w + 3) * H;
  hipLaunchKernelGGL(attn_bias_table_kernel, dim3((total + 255) / 256), dim3(256), 0,
                     as_stream(stream), table, table_rows, H, lut, w * w, tok_row_ct, tok_row_tc,
                     tok_row_tt, btab);
  return check_launch("attn_bias_table");
}

extern "C" int shrimp_attn(const shrimp_attn_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->S > 0 && a->H > 0, "attn: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->q && a->k && a->v && a->o && a->seq_lens, "attn: null pointer");
  SHRIMP_REQUIRE(a->d > 0 && a->d % 4 == 0 && a->d <= a->dpad, "attn: head dim %d / pad %d",
                 a->d, a->dpad);
  SHRIMP_REQUIRE(a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_sr % 4 == 0,
                 "attn: output strides must be multiples of 4");
  SHRIMP_REQUIRE(a->n_tokens >= 0 && a->n_tokens <= a->S, "attn: bad n_tokens");
  const int64_t extent =
      (int64_t)(a->B - 1) * a->qkv_sb + (int64_t)(a->H - 1) * a->qkv_sh + (int64_t)a->S * a->dpad;
  SHRIMP_REQUIRE(extent * 2 < (int64_t)0x7FFF0000, "attn: q/k/v buffers too large");
  const float qk_scale = SHRIMP_LOG2E / sqrtf((float)a->d);
  hipStream_t st = as_stream(stream);
  if (a->pair != nullptr) {
    SHRIMP_REQUIRE(a->table2 && a->table_rows > 0, "attn: pair mode needs table2");
    return dispatch_attn<true>(a, qk_scale, (uint32_t)(extent * 2), a->table_rows, st);
  }
  SHRIMP_REQUIRE(a->btab && a->lut_m >= 0, "attn: coords mode needs btab");
  SHRIMP_REQUIRE(a->n_tokens == a->S || (a->coords && a->mask), "attn: coords mode needs coords and mask");
  const int w = 2 * a->lut_m + 1;
  return dispatch_attn<false>(a, qk_scale, (uint32_t)(extent * 2), w * w + 3, st);
}
