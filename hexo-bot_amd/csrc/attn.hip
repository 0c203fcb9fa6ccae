// Fused relative-position-biased, key-masked attention for gfx950.
//
// Semantics: RelPosAttention's softmax(q k^T / sqrt(d) + bias) v with the
// per-block bias table (packages/shrimp/python/shrimp/model.py:448-492,
// 677-760) and the serve kernel's key bound (_triton_attn.py:59-130):
// keys >= seq_lens[b] are never visited, pad keys inside it get weight 0.
//
// One workgroup = one position x HG heads. K (key-major) and V (dim-major) of
// those heads, per-key coordinates and the heads' bias tables are staged in
// LDS once; each wave then walks 16-query blocks over 16-key blocks. All
// products stay in the "transposed" MFMA orientation so no value changes
// lanes:
//   S^T = K Q^T   (16x16x16): lane l holds keys 4*(l/16)+j of query l%16,
//                 which is the B-operand layout of P^T;
//   O^T += V^T P^T (16x16x32 over two key blocks): lane l holds dims
//                 4*(l/16)+j of query l%16, so the online-softmax rescale uses
//                 the lane's own running max;
//   row sums: one more MFMA of P^T against a constant ones row of "V^T".
// Key chunks take one of three bias paths (chosen per wave, uniformly):
//   LINEAR  positions whose live cells span <= 26 in q and r: the offset LUT
//           needs no clamping, so the bias is read at byte offset
//           kkey[key] - qkey[query] of an unclamped 53x53 fp16 table (the
//           reference also rounds the table to fp16, model.py:741). Token
//           and dead keys carry the offset code of a live cell, token
//           queries that of a live cell; blocks holding them (flagged per
//           chunk) then select the token biases / drop dead keys per lane;
//   CLAMP   all keys live cells, wider positions: clamped LUT index into the
//           fp32 table in global memory (L1/L2 resident);
//   GENERAL token rows / columns, dead keys and the key bound of wider
//           positions (and the pair tensor of the reference operator ABI).
// Softmax runs in base 2 with log2(e) folded into scale and tables; scores,
// statistics and accumulators are fp32, P enters the MFMAs as bf16.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

#define SHRIMP_LOG2E 1.4426950408889634f
#define SHRIMP_NEG_BIG (-1.0e30f)

enum : int { KEY_CELL = 0, KEY_TOKEN = 1, KEY_DEAD = 2 };
enum : int { PATH_GENERAL = 0, PATH_CLAMP = 1, PATH_LINEAR = 2 };

// Unclamped offset table: offsets with |dq|, |dr| <= XD. In memory it is head
// pair major, ((H + 1) / 2, XP, 2) fp16: each head pair's XW*XW dwords padded
// to XP, so a workgroup copies its pair's table in whole 1 KiB DMAs.
constexpr int XD = SHRIMP_ATTN_XD;
constexpr int XW = 2 * XD + 1;
constexpr int XP = SHRIMP_ATTN_XP;
static_assert(XP >= XW * XW && XP % 256 == 0, "XP: XW*XW dwords in whole 1 KiB pieces");

SHRIMP_DEV int clampi(int x, int m) { return min(max(x, -m), m); }

// LDS byte addresses as plain integers: table reads at a computed address
// then need no base pointer added per read.
typedef __attribute__((address_space(3))) const unsigned char lds_cu8;
typedef __attribute__((address_space(3))) void lds_dst_t;
SHRIMP_DEV int lds_addr(const void* p) { return (int)(uintptr_t)(lds_cu8*)p; }
SHRIMP_DEV unsigned lds_u32(int addr) {
  return *(__attribute__((address_space(3))) const unsigned*)(uintptr_t)(unsigned)addr;
}
SHRIMP_DEV float lds_f16(int addr) {
  return (float)*(__attribute__((address_space(3))) const _Float16*)(uintptr_t)(unsigned)addr;
}

// Key table of one position (shrimp_attn_keys), int32 words laid out as the
// attention kernel's LDS region that starts at kqr:
//   [kqr: 2 SP][kkey: SP][kcls: SP][blk_gen: NKB][q_gen: NKB][blk_dead: NKB][hdr: 8]
// padded to 16 bytes. kkey holds the relative LINEAR code (q XW + r) 2 HG of
// the key (token and dead keys: of the live cell (q0, r0)) for two heads per
// workgroup; hdr holds the span test and (q0, r0).
enum : int { HDR_SPAN_OK = 0, HDR_SAFE_Q = 1, HDR_SAFE_R = 2 };
__host__ __device__ inline int attn_meta_ints(int SP) {
  return (4 * SP + 3 * (SP / 16) + 8 + 3) & ~3;
}

template <int HG>
struct AttnLds {
  unsigned short* Ks;  // [HG][KD][SP/16] K fragments (256 bf16 each)
  unsigned short* Vt;  // [HG][KD][SP/16] V fragments (256 bf16 each)
  int2* kqr;           // [SP] key coordinates
  int* kkey;           // [SP] LDS byte address of the key's table row for query
                       // offset code 0: xtab + (q*XW + r + XD*XW + XD) * 2 HG
  int* kcls;           // [SP] KEY_CELL / KEY_TOKEN / KEY_DEAD
  int* blk_gen;        // [SP / 16] 1 if the block holds a token or dead key
  int* blk_dead;       // [SP / 16] 1 if the block holds a dead key (or keys past the bound)
  float* tokb;         // [3][HG] biases of (cell query, token key), (token query,
                       // cell key), (token, token), log2e folded
  float* tab;          // pair mode: [rows][HG] fp32 (log2e folded)
  _Float16* xtab;      // coords mode: [XW*XW][HG] unclamped offset table, fp16
};

struct AttnQuery {
  int query, qq, qr, qkey;  // qkey: byte offset code (q*XW + r) * 2 HG
  bool qtok, qv;
};



// One chunk of NBK 16-key blocks (NBK in {1, 2, 4}) for the HG heads of one
// 16-query block.
// LINEAR-path exceptions of a chunk (FL bits, compile time):
//   FL_QTOK  the query block holds token queries: their biases toward cell
//            keys are selected per lane;
//   FL_KTOK  the chunk's first key block holds the token keys;
//   FL_DEAD  the chunk holds dead keys (masked cells, keys past the bound):
//            they are left out of the maximum and get p = 0, so they drop out
//            of the output and the normaliser whatever their K and V rows hold
//            (finite values).
enum : int { FL_QTOK = 1, FL_KTOK = 2, FL_DEAD = 4 };

template <int DP, int HG, bool PAIR, int NBK, int PATH, int FL = 0>
SHRIMP_DEV void attn_chunk(const shrimp_attn_args& a, const AttnLds<HG>& s, const AttnQuery& qi,
                           int kb0, int L, int SP, int lr, int lg, float qk_scale, int npos,
                           const u32x2 (&qf)[HG][DP / 16], float (&m)[HG], float (&l)[HG],
                           f32x4 (&o)[HG][DP / 16]) {
  constexpr int KD = DP / 16;
  const int NKB = SP / 16;
  const int M = a.lut_m;
  const int W = 2 * M + 1;
  // this lane's K and V fragment slots of the chunk's first key block: the
  // blocks of one head follow at 512-byte steps (immediate LDS offsets)
  const unsigned short* kbase = s.Ks + kb0 * 256 + (lg * 16 + lr) * 4;
  const unsigned short* vbase = s.Vt + kb0 * 256 + (lg * 16 + lr) * 4;
  f32x4 sc4[HG][NBK];
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const u32x2 kf = *reinterpret_cast<const u32x2*>(kbase + (h * KD + kd) * NKB * 256 + kb * 256);
        acc = mfma16x16x16(kf, qf[h][kd], acc);
      }
      sc4[h][kb] = acc;
    }
  // Bias of every (key, head) of the chunk, fp32, log2e folded.
  float bias[NBK][4][HG];
  bool live[NBK][4];
  // this lane's biases toward token keys and (token queries) cell keys
  float tkb[HG], ckb[HG];
  if (FL & (FL_QTOK | FL_KTOK)) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      tkb[h] = qi.qtok ? s.tokb[2 * HG + h] : s.tokb[h];
      ckb[h] = s.tokb[HG + h];
    }
  }
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = (kb0 + kb) * 16 + lg * 4 + j;
      live[kb][j] = true;
      if (PAIR) {
        if (PATH == PATH_GENERAL) live[kb][j] = key < L;
        const uint8_t* prow = a.pair + (int64_t)blockIdx.y * a.p_sb + (int64_t)qi.query * a.p_sq;
        int p = (live[kb][j] && qi.qv) ? (int)prow[key] : 0;
        p = p < npos ? p : npos - 1;
#pragma unroll
        for (int h = 0; h < HG; ++h) bias[kb][j][h] = s.tab[p * HG + h];
      } else if (PATH == PATH_LINEAR) {
        const int xa = s.kkey[key] - qi.qkey;
        if (HG == 2) {
          const unsigned w = lds_u32(xa);
          bias[kb][j][0] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
          bias[kb][j][HG - 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
        } else {
#pragma unroll
          for (int h = 0; h < HG; ++h) bias[kb][j][h] = lds_f16(xa + 2 * h);
        }
        if (FL & FL_QTOK) {
#pragma unroll
          for (int h = 0; h < HG; ++h) bias[kb][j][h] = qi.qtok ? ckb[h] : bias[kb][j][h];
        }
        if (FL & FL_DEAD) live[kb][j] = s.kcls[key] != KEY_DEAD;
        if ((FL & FL_KTOK) && kb == 0) {
          const bool ktok = key < a.n_tokens;
#pragma unroll
          for (int h = 0; h < HG; ++h) bias[kb][j][h] = ktok ? tkb[h] : bias[kb][j][h];
        }
      } else {
        const int2 kk = s.kqr[key];
        const int p = (clampi(kk.x - qi.qq, M) + M) * W + (clampi(kk.y - qi.qr, M) + M);
        if (PATH == PATH_CLAMP) {
#pragma unroll
          for (int h = 0; h < HG; ++h) bias[kb][j][h] = a.btab[p * a.H + blockIdx.x * HG + h];
        } else {
          const int cls = s.kcls[key];
          live[kb][j] = cls != KEY_DEAD;
          const int tp = qi.qtok ? W * W + 2 : W * W;  // key token: (token | cell) query
          const int cp = qi.qtok ? W * W + 1 : p;      // key cell
          const int pp = cls == KEY_TOKEN ? tp : cp;
#pragma unroll
          for (int h = 0; h < HG; ++h) bias[kb][j][h] = a.btab[pp * a.H + blockIdx.x * HG + h];
        }
      }
    }
  // Constant A fragment: row 0 of "V^T" is all ones, so P^T times it gives the
  // per-query sum of P in accumulator row 0 (lane group 0, element 0).
  const unsigned one2 = lr == 0 ? 0x3F803F80u : 0u;
  constexpr bool MASKED = PATH == PATH_GENERAL || (PATH == PATH_LINEAR && (FL & FL_DEAD));
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    float sc[NBK][4];
    float mx = SHRIMP_NEG_BIG;
#pragma unroll
    for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = fmaf(sc4[h][kb][j], qk_scale, bias[kb][j][h]);
        if (MASKED) v = live[kb][j] ? v : SHRIMP_NEG_BIG;
        sc[kb][j] = v;
        mx = fmaxf(mx, v);
      }
    mx = max_groups_swap(mx);
    const float mnew = fmaxf(m[h], mx);
    const float alpha = __builtin_amdgcn_exp2f(m[h] - mnew);
    m[h] = mnew;
    u32x2 pf[NBK];
#pragma unroll
    for (int kb = 0; kb < NBK; ++kb) {
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[j] = __builtin_amdgcn_exp2f(sc[kb][j] - mnew);
        if (MASKED) p[j] = live[kb][j] ? p[j] : 0.f;
      }
      pf[kb].x = pack_bf16x2(p[0], p[1]);
      pf[kb].y = pack_bf16x2(p[2], p[3]);
    }
    f32x4 lacc = f32x4{l[h] * alpha, 0.f, 0.f, 0.f};
    f32x4 acc[KD];
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) acc[kd] = o[h][kd] * alpha;
    if (NBK == 1) {
      lacc = mfma16x16x16(u32x2{one2, one2}, pf[0], lacc);
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const u32x2 vf = *reinterpret_cast<const u32x2*>(vbase + (h * KD + kd) * NKB * 256);
        acc[kd] = mfma16x16x16(vf, pf[0], acc[kd]);
      }
    } else {
#pragma unroll
      for (int kp = 0; kp < NBK; kp += 2) {
        // k slots 0-3 of lane group g: keys 4g..4g+3 of block kp; 4-7: of kp+1.
        const u32x4 pp = u32x4{pf[kp].x, pf[kp].y, pf[kp + 1].x, pf[kp + 1].y};
        lacc = mfma16x16x32(u32x4{one2, one2, one2, one2}, pp, lacc);
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) {
          const unsigned short* vf = vbase + (h * KD + kd) * NKB * 256 + kp * 256;
          const u32x2 v0 = *reinterpret_cast<const u32x2*>(vf);
          const u32x2 v1 = *reinterpret_cast<const u32x2*>(vf + 256);
          acc[kd] = mfma16x16x32(u32x4{v0.x, v0.y, v1.x, v1.y}, pp, acc[kd]);
        }
      }
    }
    l[h] = lacc[0];
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) o[h][kd] = acc[kd];
  }
}

// LINEAR chunk with a fixed softmax offset. After a query block's first
// chunk (attn_chunk, which sets the running maximum m) the offset stays at
// that m: the QK^T accumulators start from cinit = -m / qk_scale, so
// fma(s, qk_scale, bias) is already score - m, and p = exp2 of it needs no
// maximum, no rescale of o and l and no lane exchange. Any fixed offset gives
// the same softmax; it only has to keep the row sums in range, so the chunk
// checks them (l < 2^64 covers overflow to inf and NaN) and returns false with
// o and l untouched when one leaves it; the caller then runs attn_chunk,
// which moves the offset. Exceptions as in attn_chunk (FL_KTOK cannot occur:
// key block 0 is always a first chunk); dead keys get p = 0, so the row-sum
// operand stays all ones.
template <int DP, int HG, int NBK, int FL>
SHRIMP_DEV bool attn_chunk_lazy(const AttnLds<HG>& s, const AttnQuery& qi, int kb0, int SP, int lr,
                                int lg, float qk_scale, const u32x2 (&qf)[HG][DP / 16],
                                const float (&cinit)[HG], float (&l)[HG],
                                f32x4 (&o)[HG][DP / 16]) {
  static_assert((FL & FL_KTOK) == 0, "token keys only in first chunks");
  constexpr int KD = DP / 16;
  const int NKB = SP / 16;
  const unsigned short* kbase = s.Ks + kb0 * 256 + (lg * 16 + lr) * 4;
  const unsigned short* vbase = s.Vt + kb0 * 256 + (lg * 16 + lr) * 4;
  f32x4 sc4[HG][NBK];
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb)
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      f32x4 acc = f32x4{cinit[h], cinit[h], cinit[h], cinit[h]};
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const u32x2 kf = *reinterpret_cast<const u32x2*>(kbase + (h * KD + kd) * NKB * 256 + kb * 256);
        acc = mfma16x16x16(kf, qf[h][kd], acc);
      }
      sc4[h][kb] = acc;
    }
  float ckb[HG];
  if (FL & FL_QTOK) {
#pragma unroll
    for (int h = 0; h < HG; ++h) ckb[h] = s.tokb[HG + h];
  }
  u32x2 pf[HG][NBK];
#pragma unroll
  for (int kb = 0; kb < NBK; ++kb) {
    const int key0 = (kb0 + kb) * 16 + lg * 4;
    int4 cls = int4{KEY_CELL, KEY_CELL, KEY_CELL, KEY_CELL};
    if (FL & FL_DEAD) cls = *reinterpret_cast<const int4*>(s.kcls + key0);
    const int4 kk = *reinterpret_cast<const int4*>(s.kkey + key0);
    const int kkv[4] = {kk.x, kk.y, kk.z, kk.w};
    const int clv[4] = {cls.x, cls.y, cls.z, cls.w};
    float p[HG][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int xa = kkv[j] - qi.qkey;
      float bias[HG];
      if (HG == 2) {
        const unsigned w = lds_u32(xa);
        bias[0] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
        bias[HG - 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
      } else {
#pragma unroll
        for (int h = 0; h < HG; ++h) bias[h] = lds_f16(xa + 2 * h);
      }
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        if (FL & FL_QTOK) bias[h] = qi.qtok ? ckb[h] : bias[h];
        p[h][j] = __builtin_amdgcn_exp2f(fmaf(sc4[h][kb][j], qk_scale, bias[h]));
        if (FL & FL_DEAD) p[h][j] = clv[j] != KEY_DEAD ? p[h][j] : 0.f;
      }
    }
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      pf[h][kb].x = pack_bf16x2(p[h][0], p[h][1]);
      pf[h][kb].y = pack_bf16x2(p[h][2], p[h][3]);
    }
  }
  // row sums first (lane group 0, element 0; other lanes hold zeros): a
  // chunk that takes one out of range returns before touching o
  const unsigned one2 = lr == 0 ? 0x3F803F80u : 0u;
  float ln[HG];
  bool bad = false;
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    f32x4 lacc = f32x4{l[h], 0.f, 0.f, 0.f};
    if (NBK == 1) {
      lacc = mfma16x16x16(u32x2{one2, one2}, pf[h][0], lacc);
    } else {
#pragma unroll
      for (int kp = 0; kp < NBK; kp += 2)
        lacc = mfma16x16x32(u32x4{one2, one2, one2, one2},
                            u32x4{pf[h][kp].x, pf[h][kp].y, pf[h][kp + 1].x, pf[h][kp + 1].y}, lacc);
    }
    ln[h] = lacc[0];
    bad |= !(ln[h] < 0x1p64f);
  }
  if (__builtin_amdgcn_ballot_w64(bad) != 0) return false;
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    l[h] = ln[h];
    if (NBK == 1) {
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const u32x2 vf = *reinterpret_cast<const u32x2*>(vbase + (h * KD + kd) * NKB * 256);
        o[h][kd] = mfma16x16x16(vf, pf[h][0], o[h][kd]);
      }
    } else {
#pragma unroll
      for (int kp = 0; kp < NBK; kp += 2) {
        const u32x4 pp = u32x4{pf[h][kp].x, pf[h][kp].y, pf[h][kp + 1].x, pf[h][kp + 1].y};
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) {
          const unsigned short* vf = vbase + (h * KD + kd) * NKB * 256 + kp * 256;
          const u32x2 v0 = *reinterpret_cast<const u32x2*>(vf);
          const u32x2 v1 = *reinterpret_cast<const u32x2*>(vf + 256);
          o[h][kd] = mfma16x16x32(u32x4{v0.x, v0.y, v1.x, v1.y}, pp, o[h][kd]);
        }
      }
    }
  }
  return true;
}

// PROJ (1 or 2): q, k and v are not read from memory but projected in the
// kernel from the block input rows p.x with the packed LN1 / q/k/v weights of
// shrimp_pack_attn_qkv (LayerNorm folded into the products, see the
// projection pass below):
//   keys / values: every wave projects its own 16-row blocks (wave + 4 j)
//     into the K and V fragments in LDS. K comes out of the weights-as-A
//     product already in K-fragment order; V, with the operands swapped
//     (rows as A, weights as B), in the transposed V-fragment order;
//   queries: the same pass leaves each of the wave's query blocks (the
//     blocks it walks later) in registers, at most PROJ_NQ per wave; waves
//     1-3 also project the last query block when it is split over the waves.
// PROJ = 2 regroups the grid so that the four head-pair workgroups of a
// position run on one XCD (workgroups are dealt to the 8 XCDs round-robin):
// the position's rows are then read from HBM into one L2, not four.
constexpr int PROJ_NQ = 5;
constexpr int PROJ_MAX_S = 4 * PROJ_NQ * 16;

// The query registers are chosen by a run-time slot with selects over the
// whole set; hiding each operand from the optimiser keeps it from folding
// the selects into an indexed (scratch memory) array.
SHRIMP_DEV u32x2 opaque2(u32x2 v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int DP, int HG, bool PAIR, int PROJ, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 ? (PROJ >= 3 ? 2 : 4) : 1) void attn_kernel(const shrimp_attn_args a, float qk_scale,
                                                   uint32_t qkv_bytes, int npos,
                                                   const shrimp_attn_proj_args p, uint32_t x_bytes,
                                                   uint32_t o_bytes) {
  // PROJ 1, 2: q/k/v projected in the kernel; 3: staged (K and V fragments
  // and the key table by DMA from shrimp_attn_qkv_kvf / shrimp_attn_keys);
  // 4: staged from K and V rows in the q layout (K permuted into fragment
  // order by the DMA, V rows transposed in LDS), key table in a.coords
  constexpr bool PJ = PROJ == 1 || PROJ == 2;
  constexpr bool STG = PROJ == 3 || PROJ == 4;
  static_assert(!PJ || (DP == 16 && HG == 2 && !PAIR && NW == 4),
                "projection covers d = 16, two heads, coords, four waves");
  static_assert(!STG || (DP == 16 && HG == 2 && !PAIR), "staged path covers d = 16, two heads, coords");
  static_assert(NW == 4 || NW == 8, "four or eight waves per workgroup");
  static_assert(HG == 1 || HG == 2, "one or two heads per workgroup");
  constexpr int NT = 64 * NW;  // threads per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int KD = DP / 16;
  if constexpr (STG) SHRIMP_PHASE_WG(0);  // phase builds: staging starts
  int b = blockIdx.y;
  int h0 = blockIdx.x * HG;
  if (PROJ == 2) {
    const int i = blockIdx.x + gridDim.x * blockIdx.y;
    const int r = i & 31;
    b = (i >> 5) * 8 + (r & 7);
    h0 = (r >> 3) * HG;
  }
  const int S = a.S;
  const int SP = (S + 15) & ~15;
  int L = a.seq_lens[b];
  SHRIMP_DCHECK(L >= 0 && L <= S, SHRIMP_DBG_SEQ_LEN);
  L = L < 0 ? 0 : (L > S ? S : L);
  const int LP = (L + 15) & ~15;
  const int nt = a.n_tokens;
  const int NC = S - nt;

  const int NKB = SP / 16;
  AttnLds<HG> s;
  s.Ks = reinterpret_cast<unsigned short*>(smem);
  s.Vt = s.Ks + HG * SP * DP;
  s.kqr = reinterpret_cast<int2*>(s.Vt + HG * DP * SP);
  s.kkey = reinterpret_cast<int*>(s.kqr + SP);
  s.kcls = s.kkey + SP;
  s.blk_gen = s.kcls + SP;
  int* q_gen = s.blk_gen + NKB;
  s.blk_dead = q_gen + NKB;
  const int* hdr = s.blk_dead + NKB;
  s.tokb = reinterpret_cast<float*>(reinterpret_cast<int*>(s.kqr) + attn_meta_ints(SP));
  int* span_red = reinterpret_cast<int*>(s.tokb + 3 * HG);  // [NW][4]
  // the tables (16-byte aligned: the offset table arrives in 16-byte DMA pieces)
  float* tail = reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(span_red + 4 * NW) + 15) &
                                         ~static_cast<uintptr_t>(15));
  s.tab = tail;
  s.xtab = reinterpret_cast<_Float16*>(tail);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int nkb = LP / 16;
  const __amdgpu_buffer_rsrc_t qrs = make_rsrc(a.q, qkv_bytes);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.k, qkv_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.v, qkv_bytes);
  const __amdgpu_buffer_rsrc_t ors = make_rsrc(a.o, o_bytes);
  const int64_t pos_base = (int64_t)b * a.qkv_sb;

  // Whole query blocks round-robin over the NW waves. When one block is left
  // over (nqb % NW == 1: 17 blocks at S = 264), it is split by key range into
  // NW parts, one per wave, instead of running whole on one wave; after a
  // barrier the partial softmax states go through LDS (over K and V, which
  // are no longer read) and wave 0 merges them.
  const int nqb = (L + 15) / 16;
  constexpr int PF = HG * (2 + 4 * KD);  // floats of one lane's partial state
  const bool split =
      nqb % NW == 1 && (NW - 1) * 64 * PF * 4 <= 2 * HG * SP * DP * 2;  // partials fit over K, V
  const int nmain = split ? nqb - 1 : nqb;

  // PROJ: row blocks this wave projects (nkb == nqb): its own blocks
  // wave + 4 j for j < nreg, then the split block's queries (waves 1-3).
  const int nreg = wave < nkb ? (nkb - wave + 3) / 4 : 0;
  const int nitems = PJ ? nreg + (split && wave > 0 ? 1 : 0) : 0;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.x, x_bytes);
  // rows of one 16-row block: lane (lr, lg) loads channels 32 ks + 8 lg .. +7
  // of row blk * 16 + lr; rows past the bound read as zeros
  auto load_x = [&](int j, u32x4 (&xf)[4]) {
    const int row = (j < nreg ? wave + 4 * j : nmain) * 16 + lr;
    const uint32_t off = row < L ? (uint32_t)(((int64_t)b * p.x_sb + (int64_t)row * p.x_sr) * 2) +
                                       (uint32_t)(lg * 16)
                                 : SHRIMP_OOB_OFFSET;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) xf[ks] = buf_load16(xrs, off + ks * 64);
  };
  u32x4 xnext[4];
  if (PJ && nitems > 0) load_x(0, xnext);

  bool linear_ok = false;
  int safe_q = 0, safe_r = 0;
  int kdelta = 0;  // subtracted from a query's LINEAR code: kkey - qkey is the table address
  if constexpr (STG) {
    // K and V fragments of the two heads (shrimp_attn_qkv_kvf: per (position,
    // head) SP/16 K fragments, then SP/16 V fragments, 512 bytes each), the
    // position's key table (a.v, shrimp_attn_keys) and the head pair's
    // offset table arrive by buffer-to-LDS DMA (no registers, no LDS store
    // instructions). Fragment pieces of keys >= S read past the buffer and
    // land as zeros.
    const int H = a.H;
    const int mbytes = attn_meta_ints(SP) * 4;
    const __amdgpu_buffer_rsrc_t mr =
        make_rsrc(PROJ == 4 ? static_cast<const void*>(a.coords) : a.v, (uint32_t)((int64_t)a.B * mbytes));
    if constexpr (PROJ == 3) {
      const __amdgpu_buffer_rsrc_t kvr = make_rsrc(a.k, (uint32_t)((int64_t)a.B * H * SP * 64));
      // fragments f = (tensor, h, kb) in LDS order, two per 1 KiB DMA
      const int nfr = 2 * HG * NKB;
      const int half = lane >> 5, sub = lane & 31;
      for (int i = wave; 2 * i < nfr; i += NW) {
        const int f = 2 * i + half;
        const int tensor = f >= HG * NKB ? 1 : 0;
        const int r = f - tensor * HG * NKB;
        const int h = r >= NKB ? 1 : 0;
        const int kb = r - h * NKB;
        // first key of this lane's 16 bytes: K slots (lg, lr), (lg, lr + 1) with
        // lr = 2 (sub % 8) hold keys lr, lr + 1; V slots hold keys 4 lg .. + 3
        const int key = kb * 16 + (tensor ? 4 * (sub >> 3) : 2 * (sub & 7));
        const uint32_t off =
            key < S ? (uint32_t)((((int64_t)b * H + h0 + h) * 2 + tensor) * SP * 32 + kb * 512 + sub * 16)
                    : SHRIMP_OOB_OFFSET;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kvr, (lds_dst_t*)(smem + i * 1024), 16, off, 0, 0, 0);
      }
    } else {
      // Only the nkb = LP / 16 key blocks the chunks read are copied.
      // K rows into fragment order one dword per lane, two DMAs per fragment:
      // DMA i fills half i % 2 of fragment (h, kb), i / 2 = h nkb + kb; its
      // dword w = 64 (i % 2) + lane is half w % 2 of slot w / 2 = 16 lg + lr,
      // i.e. K[kb*16 + lr][4 lg + 2 (w % 2) .. + 1]. Keys past the bound land
      // as zeros.
      const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.k, qkv_bytes);
      for (int i = wave; i < HG * nkb * 2; i += NW) {
        const int f = i >> 1;
        const int h = HG == 2 && f >= nkb ? 1 : 0;
        const int kb = f - h * nkb;
        const int w = (i & 1) * 64 + lane;
        const int slot = w >> 1;
        const int key = kb * 16 + (slot & 15);
        const int dim = 4 * (slot >> 4) + 2 * (w & 1);
        const uint32_t off =
            key < L ? (uint32_t)((pos_base + (int64_t)(h0 + h) * a.qkv_sh + key * 16 + dim) * 2)
                    : SHRIMP_OOB_OFFSET;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            kr, (lds_dst_t*)(smem + (h * NKB + kb) * 512 + (i & 1) * 256), 4, off, 0, 0, 0);
      }
      // V rows as they are: head h's key rows at Vt + h SP 32 bytes, 32 bytes
      // each, i.e. the 128 bytes of keys 4 g .. 4 g + 3 exactly where their
      // four-key V-fragment slots go (transposed below). One DMA is 32 keys;
      // lanes past the head's LP keys stay idle.
      const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.v, qkv_bytes);
      unsigned char* vdst = reinterpret_cast<unsigned char*>(s.Vt);
      const int vper = (LP + 31) >> 5;  // DMAs per head
      for (int i = wave; i < HG * vper; i += NW) {
        const int h = HG == 2 && i >= vper ? 1 : 0;
        const int piece = (i - h * vper) * 64 + lane;
        const int key = piece >> 1;
        const uint32_t off =
            key < L ? (uint32_t)((pos_base + (int64_t)(h0 + h) * a.qkv_sh + key * 16 + (piece & 1) * 8) * 2)
                    : SHRIMP_OOB_OFFSET;
        if (key < LP)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              vr, (lds_dst_t*)(vdst + h * SP * 32 + (i - h * vper) * 1024), 16, off, 0, 0, 0);
      }
    }
    unsigned char* mdst = reinterpret_cast<unsigned char*>(s.kqr);
    for (int i = wave; i * 1024 < mbytes; i += NW) {
      const int o = i * 1024 + lane * 16;
      if (o < mbytes)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(mr, (lds_dst_t*)(mdst + i * 1024), 16,
                                                 (uint32_t)((int64_t)b * mbytes + o), 0, 0, 0);
    }
    // the head pair's XP dwords of the pair-major table, 1 KiB per DMA
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xtab, (uint32_t)((H + 1) / 2 * XP * 4));
    unsigned char* xdst = reinterpret_cast<unsigned char*>(s.xtab);
    for (int i = wave; i * 256 < XP; i += NW)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (lds_dst_t*)(xdst + i * 1024), 16,
          (uint32_t)((h0 / 2) * XP * 4 + i * 1024 + lane * 16), 0, 0, 0);
    if (tid < 3 * HG) {
      const int W2 = (2 * a.lut_m + 1) * (2 * a.lut_m + 1);
      s.tokb[tid] = a.btab[(W2 + tid / HG) * H + h0 + tid % HG];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (PROJ == 4) {
      // V rows -> V fragments in place: one thread per four keys of one head
      // reads their rows (128 bytes) and writes their 16 slots (lg, lr), which
      // hold V[4 g + j][lr] for j = 0..3, into the same 128 bytes. Dead keys
      // (masked cells, past the bound) get zero V rows, as in the row-layout
      // path, and zero K slots, so no value a caller left there reaches the
      // products.
      for (int g = tid; g < HG * LP / 4; g += NT) {
        const int h = HG == 2 && g >= LP / 4 ? 1 : 0;
        const int key0 = (g - h * (LP / 4)) * 4;
        unsigned char* blk = reinterpret_cast<unsigned char*>(s.Vt) + h * SP * 32 + key0 * 32;
        const int4 cls = *reinterpret_cast<const int4*>(s.kcls + key0);
        const int clv[4] = {cls.x, cls.y, cls.z, cls.w};
        // K slots (lg', key0 % 16 + j) of fragment (h, key0 / 16)
        unsigned char* kfr = reinterpret_cast<unsigned char*>(s.Ks) + h * SP * 32 + (key0 >> 4) * 512;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (clv[j] == KEY_DEAD)
#pragma unroll
            for (int g2 = 0; g2 < 4; ++g2)
              *reinterpret_cast<u32x2*>(kfr + (g2 * 16 + (key0 & 15) + j) * 8) = u32x2{0u, 0u};
        u32x4 r[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            r[j][c] = *reinterpret_cast<const u32x4*>(blk + j * 32 + c * 16);
            if (clv[j] == KEY_DEAD) r[j][c] = u32x4{0u, 0u, 0u, 0u};
          }
        }
#pragma unroll
        for (int lr = 0; lr < 16; ++lr) {
          const int c = lr >> 3, d = (lr & 7) >> 1;
          const bool hi = (lr & 1) != 0;
          auto elem = [&](int j) { return hi ? r[j][c][d] >> 16 : r[j][c][d] & 0xFFFFu; };
          *reinterpret_cast<u32x2*>(blk + lr * 8) =
              u32x2{elem(0) | (elem(1) << 16), elem(2) | (elem(3) << 16)};
        }
      }
      __syncthreads();
    }
    SHRIMP_PHASE_WG(1);  // phase builds: K, V and the key table are in LDS
    linear_ok = hdr[HDR_SPAN_OK] != 0;
    safe_q = hdr[HDR_SAFE_Q];
    safe_r = hdr[HDR_SAFE_R];
    kdelta = lds_addr(s.xtab) + (XD * XW + XD) * 2 * HG;
  } else {
  // ---- global loads of the setup that nothing else depends on, issued first -----
  // coordinates and liveness of keys tid (and tid + 256 with four waves; the
  // rare keys beyond 512 are loaded where they are used)
  constexpr int KQN = 512 / NT;
  int kq[2] = {0, 0}, kr[2] = {0, 0};
  bool km[2] = {false, false};
  if (!PAIR) {
#pragma unroll
    for (int i = 0; i < KQN; ++i) {
      const int key = tid + NT * i;
      if (key >= nt && key < L) {
        const int64_t cell = (int64_t)b * NC + (key - nt);
        kq[i] = a.coords[cell * 2];
        kr[i] = a.coords[cell * 2 + 1];
        km[i] = a.mask[cell] != 0;
      }
    }
  }
  // the (XW*XW, HG) offset table of this head pair: XW*XW dwords of its pair
  // in the pair-major table, one pass
  constexpr int UX = (XW * XW + NT - 1) / NT;
  unsigned xv[UX];
  const bool xstage = !PAIR && HG == 2 && a.xtab != nullptr;
  if (xstage) {
    const unsigned* xg = static_cast<const unsigned*>(a.xtab) + (int64_t)(h0 / 2) * XP;
#pragma unroll
    for (int u = 0; u < UX; ++u) {
      const int x = tid + u * NT;
      xv[u] = x < XW * XW ? xg[x] : 0u;
    }
  }

  // ---- stage K and V in MFMA fragment order -----------------------------------
  // K fragment (h, kd, kb): lane (lr, lg) holds K[kb*16 + lr][kd*16 + 4lg .. +3];
  // V fragment (h, kd, kb): lane (lr, lg) holds V[kb*16 + 4lg .. +3][kd*16 + lr].
  // A wave's fragment read is then one contiguous 512-byte LDS block.
  // Global loads are issued U at a time per thread before their LDS stores.
  constexpr int CH = DP / 8;
  constexpr int U = 5;
  if constexpr (PROJ == 0) {
  {
    const int total = HG * LP * CH;
    for (int base = tid; base < total; base += NT * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * NT;
        const int h = HG == 2 && i >= LP * CH ? 1 : 0;  // HG <= 2: no division
        const int rem = i - h * LP * CH;
        const int key = rem / CH;
        const int ch = rem - key * CH;
        const bool ok = i < total && key < L;
        v[u] = buf_load16(krs, ok ? (uint32_t)((pos_base + (int64_t)(h0 + h) * a.qkv_sh +
                                               key * DP + ch * 8) * 2)
                                  : SHRIMP_OOB_OFFSET);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * NT;
        if (i >= total) break;
        const int h = HG == 2 && i >= LP * CH ? 1 : 0;  // HG <= 2: no division
        const int rem = i - h * LP * CH;
        const int key = rem / CH;
        const int ch = rem - key * CH;
        const int kd = ch >> 1;
        const int g0 = (ch & 1) * 2;  // lane group of dims ch*8 .. +3
        unsigned short* f = s.Ks + ((h * KD + kd) * NKB + key / 16) * 256 + (key & 15) * 4;
        *reinterpret_cast<u32x2*>(f + g0 * 64) = u32x2{v[u][0], v[u][1]};
        *reinterpret_cast<u32x2*>(f + (g0 + 1) * 64) = u32x2{v[u][2], v[u][3]};
      }
    }
  }
  {
    const int total = HG * (LP / 2) * CH;
    for (int base = tid; base < total; base += NT * U) {
      u32x4 v0[U], v1[U];
      bool d0[U], d1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * NT;
        const int h = HG == 2 && i >= (LP / 2) * CH ? 1 : 0;
        const int rem = i - h * (LP / 2) * CH;
        const int key = 2 * (rem / CH);
        const int ch = rem - (key / 2) * CH;
        const int64_t e0 = pos_base + (int64_t)(h0 + h) * a.qkv_sh + key * DP + ch * 8;
        // dead keys (past the bound, or masked cells) stage zero V rows: the
        // mask is loaded beside the rows and applied when they are stored
        const bool l0 = i < total && key < L;
        const bool l1 = i < total && key + 1 < L;
        v0[u] = buf_load16(vrs, l0 ? (uint32_t)(e0 * 2) : SHRIMP_OOB_OFFSET);
        v1[u] = buf_load16(vrs, l1 ? (uint32_t)((e0 + DP) * 2) : SHRIMP_OOB_OFFSET);
        d0[u] = !PAIR && l0 && key >= nt && !a.mask[(int64_t)b * NC + key - nt];
        d1[u] = !PAIR && l1 && key + 1 >= nt && !a.mask[(int64_t)b * NC + key + 1 - nt];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = base + u * NT;
        if (i >= total) break;
        const int h = HG == 2 && i >= (LP / 2) * CH ? 1 : 0;
        const int rem = i - h * (LP / 2) * CH;
        const int key = 2 * (rem / CH);
        const int ch = rem - (key / 2) * CH;
        if (d0[u]) v0[u] = u32x4{0u, 0u, 0u, 0u};
        if (d1[u]) v1[u] = u32x4{0u, 0u, 0u, 0u};
        // keys (key, key+1) are j, j+1 of lane group (key % 16) / 4
        unsigned short* f = s.Vt + ((h * KD + (ch >> 1)) * NKB + key / 16) * 256 +
                            ((key & 15) >> 2) * 64 + (key & 3);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int lrd = (ch & 1) * 8 + 2 * w;  // dim within the 16-dim block
          *reinterpret_cast<unsigned*>(f + lrd * 4) = (v0[u][w] & 0xFFFFu) | (v1[u][w] << 16);
          *reinterpret_cast<unsigned*>(f + (lrd + 1) * 4) = (v0[u][w] >> 16) | (v1[u][w] & 0xFFFF0000u);
        }
      }
    }
  }
  }
  // ---- key classes, coordinates, span of the live cells ----------------------------
  int qmin = 1 << 30, qmax = -(1 << 30), rmin = 1 << 30, rmax = -(1 << 30);
  if (!PAIR) {
    for (int key = tid, i = 0; key < LP; key += NT, ++i) {
      int q = 0, r = 0, cls = KEY_DEAD;  // keys past the bound (tokens too) are dead
      if (key < nt && key < L) {
        cls = KEY_TOKEN;
      } else if (key >= nt && key < L) {
        bool live;
        if (i < KQN) {
          q = i == 0 ? kq[0] : kq[1];
          r = i == 0 ? kr[0] : kr[1];
          live = i == 0 ? km[0] : km[1];
        } else {
          const int64_t cell = (int64_t)b * NC + (key - nt);
          q = a.coords[cell * 2];
          r = a.coords[cell * 2 + 1];
          live = a.mask[cell] != 0;
        }
        cls = live ? KEY_CELL : KEY_DEAD;
        if (cls == KEY_CELL) {
          qmin = min(qmin, q);
          qmax = max(qmax, q);
          rmin = min(rmin, r);
          rmax = max(rmax, r);
        }
      }
      s.kqr[key] = make_int2(q, r);
      s.kcls[key] = cls;
    }
  }
  // ---- bias tables of this head group -------------------------------------------------
  if (!PAIR && tid < 3 * HG) {
    const int W2 = (2 * a.lut_m + 1) * (2 * a.lut_m + 1);
    s.tokb[tid] = a.btab[(W2 + tid / HG) * a.H + h0 + tid % HG];
  }
  if (PAIR) {
    for (int i = tid; i < npos * HG; i += NT) {
      const int pos = i / HG;
      const int h = i - pos * HG;
      s.tab[i] = a.table2[pos * a.H + h0 + h] * SHRIMP_LOG2E;
    }
  } else if (a.xtab != nullptr) {
    const unsigned short* xg = static_cast<const unsigned short*>(a.xtab);
    if (HG == 2) {
#pragma unroll
      for (int u = 0; u < UX; ++u) {
        const int x = tid + u * NT;
        if (x < XW * XW) reinterpret_cast<unsigned*>(s.xtab)[x] = xv[u];
      }
    } else {
      // one head: its half of each dword of its pair
      const unsigned short* xh = xg + (int64_t)(h0 / 2) * XP * 2 + (h0 & 1);
      for (int i = tid; i < XW * XW * HG; i += NT) {
        const int x = i / HG;
        reinterpret_cast<unsigned short*>(s.xtab)[i] = xh[(int64_t)x * 2 + (i - x * HG)];
      }
    }
  }
  // Coordinate span of the live cells (block-wide min / max).
  if (!PAIR) {
    for (int m = 32; m >= 1; m >>= 1) {
      qmin = min(qmin, __shfl_xor(qmin, m, 64));
      qmax = max(qmax, __shfl_xor(qmax, m, 64));
      rmin = min(rmin, __shfl_xor(rmin, m, 64));
      rmax = max(rmax, __shfl_xor(rmax, m, 64));
    }
    if ((tid & 63) == 0) {
      const int w = tid >> 6;
      span_red[w * 4 + 0] = qmin;
      span_red[w * 4 + 1] = qmax;
      span_red[w * 4 + 2] = rmin;
      span_red[w * 4 + 3] = rmax;
    }
  }
  __syncthreads();
  // Per-block flags, from the staged key classes: key blocks with a token, a
  // dead key or keys past the bound; query blocks with a token or dead query.
  // One key per thread; a 16-key block is 16 lanes of one wave, so its flags
  // are 16-bit fields of wave ballots.
  for (int key0 = 0; key0 < LP; key0 += NT) {
    const int key = key0 + tid;
    bool kg = false, qg = false, kd = false;
    if (key < LP) {
      const int cls = PAIR ? KEY_CELL : s.kcls[key];
      if (key >= L) kg = kd = true;
      else if (cls != KEY_CELL || key < nt) kg = qg = true;
      if (key < L && cls == KEY_DEAD) kd = true;
    }
    const uint64_t bk = __builtin_amdgcn_ballot_w64(kg);
    const uint64_t bq = __builtin_amdgcn_ballot_w64(qg);
    const uint64_t bd = __builtin_amdgcn_ballot_w64(kd);
    if ((tid & 15) == 0 && key < LP) {
      const int sh = tid & 48;
      const int blk = key >> 4;
      s.blk_gen[blk] = ((bk >> sh) & 0xFFFFu) != 0;
      q_gen[blk] = ((bq >> sh) & 0xFFFFu) != 0;
      s.blk_dead[blk] = ((bd >> sh) & 0xFFFFu) != 0;
    }
  }
  if (!PAIR) {
    int q0 = span_red[0], q1 = span_red[1], r0 = span_red[2], r1 = span_red[3];
    for (int w = 1; w < NW; ++w) {
      q0 = min(q0, span_red[w * 4 + 0]);
      q1 = max(q1, span_red[w * 4 + 1]);
      r0 = min(r0, span_red[w * 4 + 2]);
      r1 = max(r1, span_red[w * 4 + 3]);
    }
    // LINEAR needs at least one live cell (its code stands in for token and
    // dead keys); an empty cell set gives q1 < q0 and takes the general path.
    linear_ok = a.xtab != nullptr && nt <= 16 && q0 <= q1 && (q1 - q0) <= XD && (r1 - r0) <= XD;
    // queries past the bound borrow (q0, r0): offsets to live cells stay in range
    safe_q = q0;
    safe_r = r0;
    // Linear offset code, in bytes of the (XW*XW, HG) fp16 table:
    // (dq, dr) -> ((dq + XD) * XW + (dr + XD)) * 2 HG = kkey - qkey. Token and
    // dead keys take the code of the live cell (q0, r0), so every LINEAR read
    // stays inside the table; their biases are selected afterwards.
    const int xoff = lds_addr(s.xtab);
    for (int key = tid; key < LP; key += NT) {
      const int2 kk = s.kcls[key] == KEY_CELL ? s.kqr[key] : make_int2(q0, r0);
      s.kkey[key] = xoff + (kk.x * XW + kk.y + XD * XW + XD) * 2 * HG;
    }
  }
  }  // staged / in-kernel setup
  // ---- PROJ: LayerNorm + q/k/v projection of this wave's row blocks ------------------
  // The raw bf16 rows are the MFMA operand; LayerNorm is applied to the
  // products: LN(x) W'^T + b' = rstd (x W'^T) + (b' - mean rstd cs), cs the
  // column sums of the bf16 weights. Row statistics come from packed bf16 dot
  // products (sum, sum of squares; variance = E[x^2] - mean^2 in fp32).
  // Key classes are in LDS: dead keys (masked cells, keys past the bound) get
  // zero V rows; rows past the bound zero K and Q, as the staged path reads
  // them from the zero-padded tensor.
  u32x2 qst[PROJ_NQ][HG];
  if constexpr (PJ) {
#pragma unroll
    for (int sl = 0; sl < PROJ_NQ; ++sl)
#pragma unroll
      for (int h = 0; h < HG; ++h) qst[sl][h] = u32x2{0u, 0u};
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.packed, QKV_W_BYTES);
    const float* pbias = reinterpret_cast<const float*>(static_cast<const unsigned char*>(p.packed) + QKV_B_OFF);
    const float* pcs = reinterpret_cast<const float*>(static_cast<const unsigned char*>(p.packed) + QKV_CS_OFF);
    auto wfrag = [&](int ks, int nb) {
      return buf_load16(wrs, (uint32_t)(((ks * QKV_NB + nb) * 64 + lane) * 16));
    };
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    for (int j = 0; j < nitems; ++j) {
      u32x4 xf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) xf[ks] = xnext[ks];
      if (j + 1 < nitems) load_x(j + 1, xnext);
      const bool kv = j < nreg;  // wave-uniform
      const int kb = kv ? wave + 4 * j : nmain;
      const bool rowv = kb * 16 + lr < L;
      // statistics of row lr (32 channels per lane, 4 lane groups)
      float sx = 0.f, sq = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          // element copied out first: __builtin_bit_cast of a vector element
          // (xf[ks][w] directly) reads element 0 whatever the index
          const unsigned u = xf[ks][w];
          const bf16x2 v = __builtin_bit_cast(bf16x2, u);
          sx = __builtin_amdgcn_fdot2_f32_bf16(v, ones, sx, false);
          sq = __builtin_amdgcn_fdot2_f32_bf16(v, v, sq, false);
        }
      const float mean = sum_groups_swap(sx) * (1.0f / QKV_C);
      const float var = fmaxf(sum_groups_swap(sq) * (1.0f / QKV_C) - mean * mean, 0.f);
      const float rstd = rsqrtf(var + p.eps);
      const float nmr = -mean * rstd;
      // the V fragment holds rows 4 lg + i: their statistics from lanes 4 lg + i
      float vr[4], vn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vr[i] = __shfl(rstd, lg * 4 + i, 64);
        vn[i] = __shfl(nmr, lg * 4 + i, 64);
      }
      // outputs n0 + 4 lg .. +3 of row lr (Q, K fragment order)
      auto proj_rows = [&](int n0, f32x4 acc) -> u32x2 {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(pbias + n0 + lg * 4);
        const f32x4 cc = *reinterpret_cast<const f32x4*>(pcs + n0 + lg * 4);
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = fmaf(acc[i], rstd, fmaf(nmr, cc[i], bb[i]));
        return rowv ? u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])} : u32x2{0u, 0u};
      };
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        const int hh = h0 + h;
        // queries: outputs 16 hh + 4 lg .. +3 of row lr
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(wfrag(ks, hh), xf[ks], acc);
        const u32x2 qv = proj_rows(hh * 16, acc);
#pragma unroll
        for (int sl = 0; sl < PROJ_NQ; ++sl) qst[sl][h] = sl == j ? qv : opaque2(qst[sl][h]);
        if (kv) {
          // keys: outputs QKV_C + 16 hh + 4 lg .. +3 of row lr = K-fragment order
          acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(wfrag(ks, 8 + hh), xf[ks], acc);
          *reinterpret_cast<u32x2*>(s.Ks + (h * NKB + kb) * 256 + (lg * 16 + lr) * 4) =
              proj_rows(QKV_C + hh * 16, acc);
          // values: rows 4 lg .. +3 of output 2 QKV_C + 16 hh + lr = V-fragment order
          const int nv = 2 * QKV_C + hh * 16 + lr;
          const float bv = pbias[nv], cv = pcs[nv];
          acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(xf[ks], wfrag(ks, 16 + hh), acc);
          const int4 cls = *reinterpret_cast<const int4*>(s.kcls + kb * 16 + lg * 4);
          const int cl[4] = {cls.x, cls.y, cls.z, cls.w};
          float y[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            y[i] = cl[i] != KEY_DEAD ? fmaf(acc[i], vr[i], fmaf(vn[i], cv, bv)) : 0.f;
          *reinterpret_cast<u32x2*>(s.Vt + (h * NKB + kb) * 256 + (lg * 16 + lr) * 4) =
              u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        }
      }
    }
  }
  __syncthreads();

  // One query block over key blocks [k0, k1): online-softmax state in m, l, o.
  // PROJ: the block's queries are slot `slot` of the registers filled above
  // (slot j of a wave = its block wave + 4 j; the split block's slot follows
  // the wave's own blocks).
  auto run_block = [&](int qb, int slot, int k0, int k1, AttnQuery& qi, float (&m)[HG],
                       float (&l)[HG], f32x4 (&o)[HG][KD], const u32x2 (&qin)[HG][KD]) {
    qi.query = qb * 16 + lr;
    qi.qv = qi.query < L;
    qi.qtok = qi.query < nt;
    qi.qq = 0;
    qi.qr = 0;
    qi.qkey = 0;
    if (!PAIR) {
      const int2 qc = s.kqr[qi.query];
      const bool qcell = qi.qv && !qi.qtok;
      qi.qq = qcell ? qc.x : safe_q;
      qi.qr = qcell ? qc.y : safe_r;
      qi.qkey = (qi.qq * XW + qi.qr) * 2 * HG - kdelta;
    }
    // token or dead queries in this block: general path (wave-uniform)
    const bool qgen = q_gen[qb] != 0;
    u32x2 qf[HG][KD];
    if constexpr (PJ) {
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        qf[h][0] = opaque2(qst[0][h]);
#pragma unroll
        for (int sl = 1; sl < PROJ_NQ; ++sl) qf[h][0] = slot == sl ? opaque2(qst[sl][h]) : qf[h][0];
      }
    } else {
#pragma unroll
      for (int h = 0; h < HG; ++h)
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) qf[h][kd] = qin[h][kd];
    }
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      m[h] = SHRIMP_NEG_BIG;
      l[h] = 0.f;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) o[h][kd] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

#define SHRIMP_CHUNK(NB, P) \
  attn_chunk<DP, HG, PAIR, NB, P>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, qf, m, l, o)
#define SHRIMP_CHUNK_FL(NB, F) \
  attn_chunk<DP, HG, PAIR, NB, PATH_LINEAR, F>(a, s, qi, kb, L, SP, lr, lg, qk_scale, npos, \
                                                qf, m, l, o)
#define SHRIMP_CHUNK_FLS(NB)                          \
  switch (fl) {                                       \
    case 0: SHRIMP_CHUNK_FL(NB, 0); break;            \
    case 1: SHRIMP_CHUNK_FL(NB, 1); break;            \
    case 2: SHRIMP_CHUNK_FL(NB, 2); break;            \
    case 3: SHRIMP_CHUNK_FL(NB, 3); break;            \
    case 4: SHRIMP_CHUNK_FL(NB, 4); break;            \
    case 5: SHRIMP_CHUNK_FL(NB, 5); break;            \
    case 6: SHRIMP_CHUNK_FL(NB, 6); break;            \
    default: SHRIMP_CHUNK_FL(NB, 7); break;           \
  }
#define SHRIMP_LAZY(NB, F) \
  attn_chunk_lazy<DP, HG, NB, F>(s, qi, kb, SP, lr, lg, qk_scale, qf, cinit, l, o)
#define SHRIMP_LAZY_FLS(NB)                                 \
  switch (fl) {                                             \
    case 0: ok = SHRIMP_LAZY(NB, 0); break;                 \
    case FL_QTOK: ok = SHRIMP_LAZY(NB, FL_QTOK); break;     \
    case FL_DEAD: ok = SHRIMP_LAZY(NB, FL_DEAD); break;     \
    default: ok = SHRIMP_LAZY(NB, FL_QTOK | FL_DEAD); break; \
  }
    int kb = k0;
    if (!PAIR && linear_ok) {
      // LINEAR everywhere, in runs of four key blocks; each chunk's
      // exceptions (token queries, token keys in block 0, dead keys) pick a
      // compile-time variant. The first chunk sets the softmax offset, the
      // others keep it (attn_chunk_lazy) unless their row sums leave range.
      const int qtokb = qb * 16 < nt ? FL_QTOK : 0;
      bool first = true;
      float cinit[HG];
      while (kb < k1) {
        const int run = min(4, k1 - kb);
        const int nb = run == 4 ? 4 : (run >= 2 ? 2 : 1);
        int dead = 0;
        for (int i = 0; i < nb; ++i) dead |= s.blk_dead[kb + i];
        const int fl = qtokb | (kb == 0 && nt > 0 ? FL_KTOK : 0) | (dead ? FL_DEAD : 0);
        bool ok = false;
        if (!first) {
          if (nb == 4) {
            SHRIMP_LAZY_FLS(4)
          } else if (nb == 2) {
            SHRIMP_LAZY_FLS(2)
          } else {
            SHRIMP_LAZY_FLS(1)
          }
        }
        if (!ok) {
          if (nb == 4) {
            SHRIMP_CHUNK_FLS(4)
          } else if (nb == 2) {
            SHRIMP_CHUNK_FLS(2)
          } else {
            SHRIMP_CHUNK_FLS(1)
          }
          first = false;
#pragma unroll
          for (int h = 0; h < HG; ++h) cinit[h] = -m[h] * (1.0f / qk_scale);
        }
        kb += nb;
      }
    }
#undef SHRIMP_LAZY
#undef SHRIMP_LAZY_FLS
    while (!(!PAIR && linear_ok) && kb < k1) {
      if (qgen || s.blk_gen[kb]) {
        SHRIMP_CHUNK(1, PATH_GENERAL);
        kb += 1;
        continue;
      }
      int run = 1;  // consecutive fast blocks starting at kb (up to 4)
      while (run < 4 && kb + run < k1 && !s.blk_gen[kb + run]) ++run;
      if (run == 4) SHRIMP_CHUNK(4, PATH_CLAMP);
      else if (run >= 2) SHRIMP_CHUNK(2, PATH_CLAMP);
      else SHRIMP_CHUNK(1, PATH_CLAMP);
      kb += run == 4 ? 4 : (run >= 2 ? 2 : 1);
    }
#undef SHRIMP_CHUNK
#undef SHRIMP_CHUNK_FL
#undef SHRIMP_CHUNK_FLS
  };

  // Output rows through a buffer resource, absent ones (query past the live
  // bound, channel past d, every row when !on) at an offset past it: no store
  // sits under a branch, so the wait for the next block's prefetched queries
  // counts exactly the stores issued after them (memory operations retire in
  // order).
  auto store_block = [&](const AttnQuery& qi, const float (&l)[HG], const f32x4 (&o)[HG][KD], bool on) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      // the row sum sits in lane group 0; broadcast it to the query's lanes
      const float lt = __shfl(l[h], lr, 64);
      const float inv = lt > 0.f ? 1.0f / lt : 0.f;
      const int64_t orow = (int64_t)b * a.o_sb + (int64_t)(h0 + h) * a.o_sh + (int64_t)qi.query * a.o_sr;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const int e = kd * 16 + lg * 4;
        u32x2 pk;
        pk.x = pack_bf16x2(o[h][kd][0] * inv, o[h][kd][1] * inv);
        pk.y = pack_bf16x2(o[h][kd][2] * inv, o[h][kd][3] * inv);
        const uint32_t off = on && qi.qv && e < a.d ? (uint32_t)((orow + e) * 2) : SHRIMP_OOB_OFFSET;
        __builtin_amdgcn_raw_buffer_store_b64(pk, ors, off, 0, 0);
      }
    }
  };

  // Query fragments of block qb (rows past the live bound, and every row when
  // !on, read zeros); each block's are requested one block ahead, with no
  // branch around the request.
  auto load_q = [&](int qb, bool on, u32x2 (&qf)[HG][KD]) {
    const int query = qb * 16 + lr;
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const int64_t e = pos_base + (int64_t)(h0 + h) * a.qkv_sh + query * DP + kd * 16 + lg * 4;
        qf[h][kd] = buf_load8(qrs, on && query < L ? (uint32_t)(e * 2) : SHRIMP_OOB_OFFSET);
      }
  };

  // (query blocks round-robin over the waves, the split last block: see nmain)
  // Small batches spread a position's query blocks over gridDim.z workgroups:
  // workgroup g takes the rounds g, g + Z, ... of the round-robin (each block on
  // the wave and with the key order it has with Z = 1, so the bits do not
  // change) and the last one the split block.
  const int qz = PJ ? 0 : (int)blockIdx.z, nz = PJ ? 1 : (int)gridDim.z;
  const bool tail_here = split && qz == nz - 1;
  AttnQuery qi;
  float m[HG], l[HG];
  f32x4 o[HG][KD];
  u32x2 qnext[HG][KD];
  // This wave's whole blocks are qb0, qb0 + NW nz, ... below nmain (nr of
  // them), then, where tail_here, its key range of the split block (round
  // nr). Every round issues the same requests and stores, none under a
  // branch.
  const int qb0 = wave + NW * qz;
  const int nr = qb0 < nmain ? (nmain - 1 - qb0) / (NW * nz) + 1 : 0;
  const int rounds = nr + (tail_here ? 1 : 0);
  if constexpr (!PJ) load_q(nr > 0 ? qb0 : nmain, rounds > 0, qnext);
  // as many dropped stores (distinct offsets past the resource, so none is
  // merged away) as a round issues after its prefetch: the loop is then
  // entered with the same requests in flight as from its last round, and the
  // wait for the prefetched queries counts the stores
#pragma unroll
  for (int i = 0; i < HG * KD; ++i)
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{0u, 0u}, ors, SHRIMP_OOB_OFFSET - i * 256u, 0, 0);
  for (int r = 0; r < rounds; ++r) {
    const bool tail = r == nr;
    const int qb = tail ? nmain : qb0 + r * NW * nz;
    u32x2 qcur[HG][KD];
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) qcur[h][kd] = qnext[h][kd];
    if constexpr (!PJ) load_q(r + 1 < nr ? qb + NW * nz : nmain, r + 1 < rounds, qnext);
    const int k0 = tail ? (wave * nkb) / NW : 0;
    const int k1 = tail ? ((wave + 1) * nkb) / NW : nkb;
    run_block(qb, r, k0, k1, qi, m, l, o, qcur);
    // the split block's partial state is merged below, not stored
    store_block(qi, l, o, !tail);
  }
  if (tail_here) {
    __syncthreads();  // K and V are no longer read: their LDS holds the partials
    float* part_lds = reinterpret_cast<float*>(smem) + ((wave - 1) * 64 + lane) * PF;
    if (wave > 0) {
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        part_lds[h * (2 + 4 * KD)] = m[h];
        part_lds[h * (2 + 4 * KD) + 1] = l[h];
#pragma unroll
        for (int kd = 0; kd < KD; ++kd)
#pragma unroll
          for (int j = 0; j < 4; ++j) part_lds[h * (2 + 4 * KD) + 2 + kd * 4 + j] = o[h][kd][j];
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        const float* part = reinterpret_cast<const float*>(smem) + lane * PF + h * (2 + 4 * KD);
        float mm = m[h];
#pragma unroll
        for (int p = 0; p < NW - 1; ++p) mm = fmaxf(mm, part[p * 64 * PF]);
        // parts that saw only masked keys keep m = NEG_BIG and l = 0: factor 0
        const float f0 = __builtin_amdgcn_exp2f(m[h] - mm);
        float lsum = l[h] * f0;
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) o[h][kd] = o[h][kd] * f0;
#pragma unroll
        for (int p = 0; p < NW - 1; ++p) {
          const float* src = part + p * 64 * PF;
          const float f = __builtin_amdgcn_exp2f(src[0] - mm);
          lsum += src[1] * f;
#pragma unroll
          for (int kd = 0; kd < KD; ++kd)
            o[h][kd] = o[h][kd] +
                       f32x4{src[2 + kd * 4], src[3 + kd * 4], src[4 + kd * 4], src[5 + kd * 4]} * f;
        }
        l[h] = lsum;
      }
      store_block(qi, l, o, true);
    }
  }

  // Query rows past the live bound store zeros.
  const int dq4 = a.d / 4;
  for (int i = qz == 0 ? tid : (S - L) * HG * dq4; i < (S - L) * HG * dq4; i += NT) {
    const int row = L + i / (HG * dq4);
    const int rem = i - (row - L) * HG * dq4;
    const int h = rem / dq4;
    const int e = (rem - h * dq4) * 4;
    unsigned short* orow = static_cast<unsigned short*>(a.o) + (int64_t)b * a.o_sb +
                           (int64_t)(h0 + h) * a.o_sh + (int64_t)row * a.o_sr;
    *reinterpret_cast<u32x2*>(orow + e) = u32x2{0u, 0u};
  }
  if constexpr (STG) SHRIMP_PHASE_WAVE(0);  // phase builds: this wave's stores are issued
}

// Bytes spanned by the output rows (a.o); callers have checked them against
// the 32-bit buffer-offset limit (attn_out_fits).
static int64_t attn_out_extent(const shrimp_attn_args* a) {
  return ((int64_t)(a->B - 1) * a->o_sb + (int64_t)(a->H - 1) * a->o_sh + (int64_t)(a->S - 1) * a->o_sr +
          a->d) * 2;
}
static bool attn_out_fits(const shrimp_attn_args* a) {
  return strides_ok({a->o_sb, a->o_sh, a->o_sr}) && attn_out_extent(a) < (int64_t)0x7FFF0000;
}
static uint32_t attn_out_bytes(const shrimp_attn_args* a) { return (uint32_t)attn_out_extent(a); }

// LDS bytes of one workgroup; npos = pair-table rows (pair mode only).
static size_t attn_smem_bytes(int DP, int HG, int S, int npos, bool pair) {
  const size_t SP = (size_t)((S + 15) & ~15);
  size_t bytes = 2 * HG * SP * DP * 2 + (size_t)attn_meta_ints((int)SP) * 4 + 3 * HG * 4 + 4 * 8 * 4;
  bytes += 16;  // alignment of the tables
  bytes += pair ? (size_t)npos * HG * 4 : (size_t)(HG == 2 ? XP : XW * XW) * HG * 2;
  return bytes;
}

template <int DP, int HG, bool PAIR, int NW>
static int launch_attn(const shrimp_attn_args* a, float qk_scale, uint32_t qkv_bytes, int npos,
                       size_t smem, hipStream_t st) {
  // query splits (small batches): up to 4, doubling while the workgroups stay
  // within two per compute unit and each split keeps at least two rounds of
  // NW query blocks
  const int groups = a->H / HG * a->B;
  const int rounds = ((a->S + 15) / 16) / NW;
  int z = 1;
  while (z < 4 && groups * z * 2 <= 2 * cu_count() && rounds >= 2 * z) z *= 2;
  dim3 grid(a->H / HG, a->B, z);
  const shrimp_attn_proj_args none{};
  hipLaunchKernelGGL((attn_kernel<DP, HG, PAIR, 0, NW>), grid, dim3(64 * NW), smem, st, *a,
                     qk_scale, qkv_bytes, npos, none, 0u, attn_out_bytes(a));
  return check_launch("attn");
}

// LDS budget per workgroup kept at 64 KiB so several groups share a CU;
// sequences too long for it take one head per workgroup with up to the
// device's per-workgroup LDS, and longer ones the chunked kernel of f32.hip
// (keys streamed through LDS, one query row per thread).
static const size_t kAttnSmemCap = 64 * 1024;
int attn_rows_bf16(const shrimp_attn_args* a, hipStream_t st);

template <bool PAIR>
static int dispatch_attn(const shrimp_attn_args* a, float qk_scale, uint32_t qkv_bytes, int npos,
                         int tab_rows, hipStream_t st) {
  if (g_attn_variant == 3) return attn_rows_bf16(a, st);
#define SHRIMP_ATTN_DP(DPV)                                                                \
  if (a->dpad == DPV) {                                                                    \
    const size_t s2 = attn_smem_bytes(DPV, 2, a->S, tab_rows, PAIR);                       \
    const size_t s1 = attn_smem_bytes(DPV, 1, a->S, tab_rows, PAIR);                       \
    if (a->H % 2 == 0 && s2 <= kAttnSmemCap && g_attn_variant != 1)                       \
      return DPV == 16 && g_attn_variant == 0                                              \
                 ? launch_attn<DPV, 2, PAIR, DPV == 16 ? 8 : 4>(a, qk_scale, qkv_bytes, npos, s2, st) \
                 : launch_attn<DPV, 2, PAIR, 4>(a, qk_scale, qkv_bytes, npos, s2, st);     \
    if (s1 <= kAttnSmemCap || s1 <= (size_t)max_lds_per_block())                          \
      return launch_attn<DPV, 1, PAIR, 4>(a, qk_scale, qkv_bytes, npos, s1, st);          \
    return attn_rows_bf16(a, st);                                                          \
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
  SHRIMP_DCHECK(row < table_rows, SHRIMP_DBG_TABLE_ROW);
  row = row < table_rows ? row : table_rows - 1;
  btab[i] = table[row * H + h] * SHRIMP_LOG2E;
}

// xtab[p, x, j] = fp16(btab[clamped LUT position of (dq, dr), 2 p + j]), x over
// the unclamped (2 XD + 1)^2 offsets; the padding (x >= XW*XW) and the missing
// second head of an odd H are zeros.
__global__ void attn_xtab_kernel(const float* __restrict__ btab, int H, int M,
                                 unsigned short* __restrict__ xtab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (H + 1) / 2 * XP * 2) return;
  const int p = i / (XP * 2);
  const int rem = i - p * XP * 2;
  const int x = rem >> 1;
  const int h = 2 * p + (rem & 1);
  float v = 0.f;
  if (x < XW * XW && h < H) {
    const int dq = x / XW - XD;
    const int dr = x - (x / XW) * XW - XD;
    const int W = 2 * M + 1;
    const int pos = (clampi(dq, M) + M) * W + (clampi(dr, M) + M);
    v = btab[pos * H + h];
  }
  xtab[i] = __builtin_bit_cast(unsigned short, (_Float16)v);
}

// Key table of every position for the staged attention (layout at
// attn_meta_ints): the classes, coordinates, LINEAR codes, per-block flags
// and span of the in-kernel setup, once per forward instead of once per
// (position, head pair, attention block). One workgroup per position; when
// `tokens` is given it also writes the position's token rows (as
// fill_tokens_kernel does) before its key work.
__global__ __launch_bounds__(256) void attn_keys_kernel(const int32_t* __restrict__ coords,
                                                        const uint8_t* __restrict__ mask,
                                                        const int32_t* __restrict__ seq_lens, int S,
                                                        int nt, int* __restrict__ meta,
                                                        const float* __restrict__ tokens, int C,
                                                        unsigned short* __restrict__ seq,
                                                        int64_t seq_sb,
                                                        unsigned short* __restrict__ tok_lo,
                                                        int vec4) {
  extern __shared__ int ks[];  // [3][SP]: class, q, r
  __shared__ int red[4][4];
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tokens) fill_token_rows(b, tokens, nt, C, seq, seq_sb, tok_lo, vec4);
  const int SP = (S + 15) & ~15, NKB = SP / 16, NC = S - nt;
  int L = seq_lens[b];
  SHRIMP_DCHECK(L >= 0 && L <= S, SHRIMP_DBG_SEQ_LEN);
  L = L < 0 ? 0 : (L > S ? S : L);
  const int mi = attn_meta_ints(SP);
  int* m = meta + (int64_t)b * mi;
  int* kkey = m + 2 * SP;
  int* kcls = m + 3 * SP;
  int* bgen = m + 4 * SP;
  int* qgen = bgen + NKB;
  int* bdead = qgen + NKB;
  int* hdr = bdead + NKB;
  int qmin = 1 << 30, qmax = -(1 << 30), rmin = 1 << 30, rmax = -(1 << 30);
  for (int key = tid; key < SP; key += 256) {
    int q = 0, r = 0, cls = KEY_DEAD;  // keys past the bound (tokens too) are dead
    if (key < nt && key < L) {
      cls = KEY_TOKEN;
    } else if (key >= nt && key < L) {
      const int64_t cell = (int64_t)b * NC + (key - nt);
      q = coords[cell * 2];
      r = coords[cell * 2 + 1];
      cls = mask[cell] != 0 ? KEY_CELL : KEY_DEAD;
      if (cls == KEY_CELL) {
        qmin = min(qmin, q);
        qmax = max(qmax, q);
        rmin = min(rmin, r);
        rmax = max(rmax, r);
      }
    }
    m[2 * key] = q;
    m[2 * key + 1] = r;
    kcls[key] = cls;
    ks[key] = cls;
    ks[SP + key] = q;
    ks[2 * SP + key] = r;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    qmin = min(qmin, __shfl_xor(qmin, o, 64));
    qmax = max(qmax, __shfl_xor(qmax, o, 64));
    rmin = min(rmin, __shfl_xor(rmin, o, 64));
    rmax = max(rmax, __shfl_xor(rmax, o, 64));
  }
  if ((tid & 63) == 0) {
    red[tid >> 6][0] = qmin;
    red[tid >> 6][1] = qmax;
    red[tid >> 6][2] = rmin;
    red[tid >> 6][3] = rmax;
  }
  __syncthreads();
  int q0 = red[0][0], q1 = red[0][1], r0 = red[0][2], r1 = red[0][3];
  for (int w = 1; w < 4; ++w) {
    q0 = min(q0, red[w][0]);
    q1 = max(q1, red[w][1]);
    r0 = min(r0, red[w][2]);
    r1 = max(r1, red[w][3]);
  }
  // LINEAR needs a live cell (its code stands in for token and dead keys)
  const bool span_ok = nt <= 16 && q0 <= q1 && (q1 - q0) <= XD && (r1 - r0) <= XD;
  // key blocks with a token, a dead key or keys past the bound; query blocks
  // with a token or dead query; key blocks with a dead key or keys past the bound
  for (int blk = tid; blk < NKB; blk += 256) {
    int kg = 0, qg = 0, kd = 0;
    for (int j = 0; j < 16; ++j) {
      const int key = blk * 16 + j;
      const int cls = ks[key];
      if (key >= L) kg = kd = 1;
      else if (cls != KEY_CELL || key < nt) kg = qg = 1;
      if (key < L && cls == KEY_DEAD) kd = 1;
    }
    bgen[blk] = kg;
    qgen[blk] = qg;
    bdead[blk] = kd;
  }
  for (int key = tid; key < SP; key += 256) {
    const bool cell = ks[key] == KEY_CELL;
    kkey[key] = span_ok ? ((cell ? ks[SP + key] : q0) * XW + (cell ? ks[2 * SP + key] : r0)) * 4 : 0;
  }
  for (int i = tid; i < mi - (4 * SP + 3 * NKB); i += 256)
    hdr[i] = i == HDR_SPAN_OK ? (int)span_ok : (i == HDR_SAFE_Q ? q0 : (i == HDR_SAFE_R ? r0 : 0));
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_attn_bias_table(const float* table, int table_rows, int H,
                                      const uint8_t* lut, int lut_m, int tok_row_ct,
                                      int tok_row_tc, int tok_row_tt, float* btab, void* xtab,
                                      void* stream) {
  SHRIMP_REQUIRE(table && lut && btab, "attn_bias_table: null pointer");
  SHRIMP_REQUIRE(table_rows > 0 && table_rows <= kMaxDim && H > 0 && H <= 1024 && lut_m >= 0 &&
                     lut_m <= 64,
                 "attn_bias_table: bad sizes (rows %d, H %d, lut_m %d)", table_rows, H, lut_m);
  SHRIMP_REQUIRE(tok_row_ct >= 0 && tok_row_ct < table_rows && tok_row_tc >= 0 &&
                     tok_row_tc < table_rows && tok_row_tt >= 0 && tok_row_tt < table_rows,
                 "attn_bias_table: token rows (%d, %d, %d) outside the %d table rows", tok_row_ct,
                 tok_row_tc, tok_row_tt, table_rows);
  const int w = 2 * lut_m + 1;
  const int total = (w * w + 3) * H;
  hipLaunchKernelGGL(attn_bias_table_kernel, dim3((total + 255) / 256), dim3(256), 0,
                     as_stream(stream), table, table_rows, H, lut, w * w, tok_row_ct, tok_row_tc,
                     tok_row_tt, btab);
  if (xtab != nullptr) {
    const int nx = (H + 1) / 2 * XP * 2;
    hipLaunchKernelGGL(attn_xtab_kernel, dim3((nx + 255) / 256), dim3(256), 0, as_stream(stream),
                       btab, H, lut_m, static_cast<unsigned short*>(xtab));
  }
  return check_launch("attn_bias_table");
}

extern "C" int shrimp_attn(const shrimp_attn_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->S > 0 && a->S <= kMaxDim && a->H > 0 && a->H <= kMaxDim,
                 "attn: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->q && a->k && a->v && a->o && a->seq_lens, "attn: null pointer");
  SHRIMP_REQUIRE(a->d > 0 && a->d % 4 == 0 && a->d <= a->dpad, "attn: head dim %d / pad %d",
                 a->d, a->dpad);
  SHRIMP_REQUIRE(a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_sr % 4 == 0,
                 "attn: output strides must be multiples of 4");
  SHRIMP_REQUIRE(attn_out_fits(a), "attn: output buffer too large");
  SHRIMP_REQUIRE(a->n_tokens >= 0 && a->n_tokens <= a->S, "attn: bad n_tokens");
  SHRIMP_REQUIRE(strides_ok({a->qkv_sb, a->qkv_sh, a->p_sb, a->p_sq}), "attn: strides outside [0, 2^31)");
  const int64_t extent =
      (int64_t)(a->B - 1) * a->qkv_sb + (int64_t)(a->H - 1) * a->qkv_sh + (int64_t)a->S * a->dpad;
  SHRIMP_REQUIRE(extent * 2 < (int64_t)0x7FFF0000, "attn: q/k/v buffers too large");
  const float qk_scale = SHRIMP_LOG2E / sqrtf((float)a->d);
  hipStream_t st = as_stream(stream);
  if (a->pair != nullptr) {
    SHRIMP_REQUIRE(a->table2 && a->table_rows > 0, "attn: pair mode needs table2");
    return dispatch_attn<true>(a, qk_scale, (uint32_t)(extent * 2), a->table_rows,
                               a->table_rows, st);
  }
  SHRIMP_REQUIRE(a->btab && a->lut_m >= 0 && a->lut_m <= 64, "attn: coords mode needs btab");
  SHRIMP_REQUIRE(a->n_tokens == a->S || (a->coords && a->mask), "attn: coords mode needs coords and mask");
  const int w = 2 * a->lut_m + 1;
  return dispatch_attn<false>(a, qk_scale, (uint32_t)(extent * 2), w * w + 3, w * w, st);
}

extern "C" int shrimp_attn_fused_supported(int C, int H, int S, int dpad) {
  return C == QKV_C && H == 8 && dpad == 16 && S > 0 && S <= PROJ_MAX_S &&
         attn_smem_bytes(16, 2, S, 0, false) <= kAttnSmemCap;
}

extern "C" int shrimp_attn_fused(const shrimp_attn_args* a, const shrimp_attn_proj_args* p,
                                 void* stream) {
  SHRIMP_REQUIRE(a != nullptr && p != nullptr, "attn_fused: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->S > 0 && a->S <= kMaxDim && a->H > 0 && a->H <= kMaxDim,
                 "attn_fused: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  const long long fc = (long long)a->H * a->d;
  SHRIMP_REQUIRE(fc == QKV_C && shrimp_attn_fused_supported(QKV_C, a->H, a->S, a->dpad),
                 "attn_fused: covers C = %d, H = 8, dpad = 16, S <= %d (got C = %lld, H = %d, "
                 "dpad = %d, S = %d)", QKV_C, PROJ_MAX_S, fc, a->H, a->dpad, a->S);
  SHRIMP_REQUIRE(a->pair == nullptr, "attn_fused: coords mode only");
  SHRIMP_REQUIRE(a->o && a->seq_lens && p->x && p->packed, "attn_fused: null pointer");
  SHRIMP_REQUIRE(a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_sr % 4 == 0,
                 "attn_fused: output strides must be multiples of 4");
  SHRIMP_REQUIRE(attn_out_fits(a), "attn: output buffer too large");
  SHRIMP_REQUIRE(a->n_tokens >= 0 && a->n_tokens <= a->S, "attn_fused: bad n_tokens");
  SHRIMP_REQUIRE(a->btab && a->lut_m >= 0 && a->lut_m <= 64, "attn_fused: needs btab");
  SHRIMP_REQUIRE(a->n_tokens == a->S || (a->coords && a->mask),
                 "attn_fused: needs coords and mask");
  SHRIMP_REQUIRE(strides_ok({p->x_sb, p->x_sr}), "attn_fused: x strides outside [0, 2^31)");
  SHRIMP_REQUIRE(p->x_sr >= QKV_C && p->x_sr % 8 == 0 && p->x_sb % 8 == 0 &&
                     p->x_sb >= (int64_t)(a->S - 1) * p->x_sr + QKV_C,
                 "attn_fused: x strides (row %lld, position %lld)", (long long)p->x_sr,
                 (long long)p->x_sb);
  const int64_t xe = ((int64_t)(a->B - 1) * p->x_sb + (int64_t)(a->S - 1) * p->x_sr + QKV_C) * 2;
  SHRIMP_REQUIRE(xe < (int64_t)0x7FFF0000, "attn_fused: input rows too large");
  const int w = 2 * a->lut_m + 1;
  const size_t smem = attn_smem_bytes(16, 2, a->S, w * w + 3, false);
  const float qk_scale = SHRIMP_LOG2E / sqrtf((float)a->d);
  dim3 grid(a->H / 2, a->B);
  // the XCD grouping needs whole groups of 8 positions (grid.x = 4 head pairs)
  if (a->B % 8 == 0)
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 2, 4>), grid, dim3(256), smem, as_stream(stream),
                       *a, qk_scale, 0u, w * w, *p, (uint32_t)xe, attn_out_bytes(a));
  else
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 1, 4>), grid, dim3(256), smem, as_stream(stream),
                       *a, qk_scale, 0u, w * w, *p, (uint32_t)xe, attn_out_bytes(a));
  return check_launch("attn_fused");
}

namespace shrimp {
int attn_phase_set(void* stamps, int cycles) {
#if SHRIMP_PHASE_CLOCK
  return phase_set(stamps, cycles);
#else
  (void)stamps;
  (void)cycles;
  return set_error(SHRIMP_EINVAL, "phase_clock: phase stamps need the phase build (SHRIMP_PHASE_CLOCK=1)");
#endif
}
}  // namespace shrimp

extern "C" size_t shrimp_attn_keys_bytes(int S) {
  return S > 0 && S <= kMaxDim ? (size_t)attn_meta_ints((S + 15) & ~15) * 4 : 0;
}

extern "C" int shrimp_attn_keys(const int32_t* coords, const uint8_t* mask, const int32_t* seq_lens,
                                int B, int S, int n_tokens, int32_t* meta, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && S > 0 && S <= 4096 && n_tokens >= 0 && n_tokens <= S,
                 "attn_keys: bad shape (S = %d, at most 4096)", S);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(seq_lens && meta && (n_tokens == S || (coords && mask)), "attn_keys: null pointer");
  const int SP = (S + 15) & ~15;
  SHRIMP_REQUIRE(SP <= 4096, "attn_keys: S = %d too large", S);
  hipLaunchKernelGGL(attn_keys_kernel, dim3(B), dim3(256), (size_t)3 * SP * 4, as_stream(stream),
                     coords, mask, seq_lens, S, n_tokens, meta, nullptr, 0, nullptr, (int64_t)0,
                     nullptr, 0);
  return check_launch("attn_keys");
}

extern "C" int shrimp_attn_keys_tokens(const int32_t* coords, const uint8_t* mask,
                                       const int32_t* seq_lens, int B, int S, int n_tokens,
                                       int32_t* meta, const float* tokens, int C, void* seq,
                                       int64_t seq_sb, void* tok_lo, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && S > 0 && S <= 4096 && n_tokens >= 0 && n_tokens <= S,
                 "attn_keys_tokens: bad shape (S = %d, at most 4096)", S);
  SHRIMP_REQUIRE(seq_lens && meta && (n_tokens == S || (coords && mask)),
                 "attn_keys_tokens: null pointer");
  const int vec4 = fill_tokens_check(tokens, n_tokens, C, seq, seq_sb, tok_lo, B);
  if (vec4 < 0) return vec4;
  if (B == 0) return SHRIMP_OK;
  const int SP = (S + 15) & ~15;
  hipLaunchKernelGGL(attn_keys_kernel, dim3(B), dim3(256), (size_t)3 * SP * 4, as_stream(stream),
                     coords, mask, seq_lens, S, n_tokens, meta, tokens, C,
                     static_cast<unsigned short*>(seq), seq_sb, static_cast<unsigned short*>(tok_lo),
                     vec4);
  return check_launch("attn_keys_tokens");
}

// The staged kernel runs four waves per workgroup while its LDS fits the
// 64 KiB budget (three workgroups per compute unit), and eight waves with the
// unit's LDS to itself past it (two waves per SIMD, up to 256 registers each):
// supports of 368 cells and more, as the evaluator pads spec-sized positions.
extern "C" int shrimp_attn_staged_supported(int H, int S, int dpad) {
  if (S <= 0 || S > 1024) return 0;
  const int SP = (S + 15) & ~15;
  return dpad == 16 && H > 0 && H % 2 == 0 && S > 0 && S % 4 == 0 && SP <= 1024 &&
         attn_smem_bytes(16, 2, S, 0, false) <= (size_t)max_lds_per_block();
}

extern "C" int shrimp_attn_staged(const shrimp_attn_args* a, const void* kvf, const int32_t* meta,
                                  void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_staged: null args");
  SHRIMP_REQUIRE(a->B >= 0 && a->S > 0 && a->H > 0, "attn_staged: bad shape");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(shrimp_attn_staged_supported(a->H, a->S, a->dpad),
                 "attn_staged: covers dpad = 16, even H, S %% 4 == 0 (got H = %d, S = %d, dpad = %d)",
                 a->H, a->S, a->dpad);
  SHRIMP_REQUIRE(a->pair == nullptr, "attn_staged: coords mode only");
  // kvf NULL: K and V rows from a->k, a->v in the layout of a->q
  const bool rows = kvf == nullptr;
  SHRIMP_REQUIRE(a->q && meta && a->o && a->seq_lens && a->btab && a->xtab && (!rows || (a->k && a->v)),
                 "attn_staged: null pointer");
  SHRIMP_REQUIRE(a->d > 0 && a->d % 4 == 0 && a->d <= 16, "attn_staged: head dim %d", a->d);
  SHRIMP_REQUIRE(a->o_sb % 4 == 0 && a->o_sh % 4 == 0 && a->o_sr % 4 == 0,
                 "attn_staged: output strides must be multiples of 4");
  SHRIMP_REQUIRE(attn_out_fits(a), "attn: output buffer too large");
  SHRIMP_REQUIRE(a->n_tokens >= 0 && a->n_tokens <= a->S, "attn_staged: bad n_tokens");
  SHRIMP_REQUIRE(a->lut_m >= 0 && a->lut_m <= 64, "attn_staged: lut_m");
  const int SP = (a->S + 15) & ~15;
  SHRIMP_REQUIRE(strides_ok({a->qkv_sb, a->qkv_sh}), "attn_staged: q strides outside [0, 2^31)");
  const int64_t kvb = mul_sat({a->B, a->H, SP, 64});
  const int64_t mb = mul_sat({a->B, (int64_t)shrimp_attn_keys_bytes(a->S)});
  const int64_t qe = ((int64_t)(a->B - 1) * a->qkv_sb + (int64_t)(a->H - 1) * a->qkv_sh +
                      (int64_t)a->S * a->dpad) * 2;
  SHRIMP_REQUIRE(kvb < (int64_t)0x7FFF0000 && mb < (int64_t)0x7FFF0000 && qe < (int64_t)0x7FFF0000,
                 "attn_staged: buffers too large");
  shrimp_attn_args s = *a;
  if (rows) {
    s.coords = meta;
  } else {
    s.k = kvf;
    s.v = meta;
  }
  const float qk_scale = SHRIMP_LOG2E / sqrtf((float)a->d);
  const size_t smem = attn_smem_bytes(16, 2, a->S, 0, false);
  // four waves per workgroup (three workgroups per compute unit): measured
  // faster than eight where the 64 KiB budget holds; past it eight waves
  const bool big = smem > kAttnSmemCap;
  const int NW = big ? 8 : 4;
  const int groups = a->H / 2 * a->B;
  const int rounds = ((a->S + 15) / 16) / NW;
  int z = 1;
  while (z < 4 && groups * z * 2 <= 2 * cu_count() && rounds >= 2 * z) z *= 2;
  dim3 grid(a->H / 2, a->B, z);
  const shrimp_attn_proj_args none{};
  if (rows && big)
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 4, 8>), grid, dim3(64 * 8), smem,
                       as_stream(stream), s, qk_scale, (uint32_t)qe, 0, none, 0u, attn_out_bytes(a));
  else if (rows)
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 4, 4>), grid, dim3(64 * 4), smem,
                       as_stream(stream), s, qk_scale, (uint32_t)qe, 0, none, 0u, attn_out_bytes(a));
  else if (big)
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 3, 8>), grid, dim3(64 * 8), smem,
                       as_stream(stream), s, qk_scale, (uint32_t)qe, 0, none, 0u, attn_out_bytes(a));
  else
    hipLaunchKernelGGL((attn_kernel<16, 2, false, 3, 4>), grid, dim3(64 * 4), smem,
                       as_stream(stream), s, qk_scale, (uint32_t)qe, 0, none, 0u, attn_out_bytes(a));
  return check_launch("attn_staged");
}
