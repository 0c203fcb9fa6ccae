// Shared device helpers for the Shrimp gfx950 kernels.
//
// Conventions used by every kernel in this directory:
//  * wave64; MFMA operands follow the CDNA lane layouts: for a 16x16xK tile
//    lane l supplies row/col (l % 16) and the K slice owned by lane group
//    (l / 16); the 16x16 f32 result gives lane l rows 4*(l/16)+j (j=0..3) of
//    column (l % 16).
//  * activations are bf16, accumulation and all statistics fp32.
//  * gathered reads go through buffer resources: an offset past the record
//    count returns zeros, so a missing neighbour (index >= N) is a zero row
//    by construction and no gathered read can leave its buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

#define SHRIMP_DEV __device__ __forceinline__

// Buffer resource word 3 for gfx9-family raw buffers (no format conversion).
#define SHRIMP_RSRC_W3 0x00020000

// Offset used for "absent" rows: far past any record count.
#define SHRIMP_OOB_OFFSET 0x7FFFFF00u

SHRIMP_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           SHRIMP_RSRC_W3);
}

SHRIMP_DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}
SHRIMP_DEV u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0);
}
SHRIMP_DEV unsigned buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
}

// ---- input checks of checked builds (SHRIMP_DEBUG=1) ---------------------------
//
// SHRIMP_DCHECK(cond, bit) compiles to nothing in release builds. In checked
// builds a failed condition sets `bit` in this source file's device fault word
// (a relaxed device-scope atomic OR; the kernel then goes on exactly as a
// release build does, so an absent row still reads zeros), and the launch
// wrapper's check_launch synchronises and reports the word as SHRIMP_ECHECK.
// The index checks follow the reference kernels' contract: an index at or past
// the rows is absent (their `idx < Npad` test), -1 is absent here too, and a
// more negative one would gather before the rows there.
#define SHRIMP_DBG_CONV_INDEX 0x1u  // conv neighbour index below -1
#define SHRIMP_DBG_SEQ_LEN 0x2u     // sequence length outside [0, S]
#define SHRIMP_DBG_RAY_INDEX 0x4u   // ray-tap / gather index below -1
#define SHRIMP_DBG_LEGAL 0x8u       // legal count outside [0, row]
#define SHRIMP_DBG_NBR 0x10u        // packed neighbour id neither absent nor in the row
#define SHRIMP_DBG_TABLE_ROW 0x20u  // bias LUT entry past the bias table's rows

#if SHRIMP_DEBUG
namespace shrimp {
static __device__ unsigned g_debug_fault;

SHRIMP_DEV void debug_fault(unsigned bit) {
  __hip_atomic_fetch_or(&g_debug_fault, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static int debug_sync(const char* what) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return set_error(SHRIMP_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  unsigned f = 0;
  e = hipMemcpyFromSymbol(&f, HIP_SYMBOL(g_debug_fault), sizeof(f));
  if (e != hipSuccess) return set_error(SHRIMP_ELAUNCH, "%s: fault word: %s", what, hipGetErrorString(e));
  if (f == 0) return SHRIMP_OK;
  const unsigned zero = 0;
  (void)hipMemcpyToSymbol(HIP_SYMBOL(g_debug_fault), &zero, sizeof(zero));
  return set_error(SHRIMP_ECHECK, "%s: input checks failed (0x%x:%s%s%s%s%s%s)", what, f,
                   (f & SHRIMP_DBG_CONV_INDEX) ? " conv index" : "",
                   (f & SHRIMP_DBG_SEQ_LEN) ? " sequence length" : "",
                   (f & SHRIMP_DBG_RAY_INDEX) ? " ray/gather index" : "",
                   (f & SHRIMP_DBG_LEGAL) ? " legal count" : "",
                   (f & SHRIMP_DBG_NBR) ? " neighbour id" : "",
                   (f & SHRIMP_DBG_TABLE_ROW) ? " bias table row" : "");
}
}  // namespace shrimp
#define SHRIMP_DCHECK(cond, bit)                  \
  do {                                            \
    if (!(cond)) ::shrimp::debug_fault(bit);      \
  } while (0)
#else
#define SHRIMP_DCHECK(cond, bit) ((void)0)
#endif

// ---- phase stamps of measurement builds (SHRIMP_PHASE_CLOCK=1) -----------------
//
// SHRIMP_PHASE_WG(slot) and SHRIMP_PHASE_WAVE(k) compile to nothing in other
// builds. In a phase build, while shrimp_phase_clock has set a stamp buffer
// for the source file's kernels, they store the 100 MHz constant clock
// (s_memrealtime) into 32 u64 slots per workgroup (workgroup blockIdx.x +
// gridDim.x blockIdx.y; blockIdx.z is not told apart): slots 0-7 from thread 0
// at workgroup-wide points (after a barrier), and when asked for, each with the
// core clock counter (s_memtime) at slot + 8, so a phase's cycles over its wall
// time give the clock the compute unit ran at (a second counter read per stamp,
// so timings are taken from runs without it); slot 16 + 8 k + wave from lane 0
// of each wave (k = 0, 1; waves < 8).
#ifndef SHRIMP_PHASE_CLOCK
#define SHRIMP_PHASE_CLOCK 0
#endif
#if SHRIMP_PHASE_CLOCK
namespace shrimp {
static __device__ unsigned long long* g_phase_buf;
static __device__ int g_phase_cycles;

static int phase_set(void* buf, int cycles) {
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_phase_buf), &buf, sizeof(buf));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_phase_cycles), &cycles, sizeof(cycles));
  return e == hipSuccess ? SHRIMP_OK : set_error(SHRIMP_ELAUNCH, "phase_clock: %s", hipGetErrorString(e));
}

SHRIMP_DEV void phase_stamp(int slot, bool writer) {
  unsigned long long* p = g_phase_buf;
  if (p != nullptr && writer) {
    unsigned long long* w = p + (size_t)(blockIdx.x + gridDim.x * blockIdx.y) * 32;
    w[slot] = __builtin_amdgcn_s_memrealtime();
    if (slot < 8 && g_phase_cycles) w[slot + 8] = __builtin_amdgcn_s_memtime();
  }
}
}  // namespace shrimp
#define SHRIMP_PHASE_WG(slot) ::shrimp::phase_stamp((slot), threadIdx.x == 0)
#define SHRIMP_PHASE_WAVE(k) \
  ::shrimp::phase_stamp(16 + 8 * (k) + (int)(threadIdx.x >> 6), (threadIdx.x & 63) == 0)
#else
#define SHRIMP_PHASE_WG(slot) ((void)0)
#define SHRIMP_PHASE_WAVE(k) ((void)0)
#endif

// ---- bf16 <-> f32 -----------------------------------------------------------

SHRIMP_DEV float bf16_lo(unsigned w) { return __uint_as_float(w << 16); }
SHRIMP_DEV float bf16_hi(unsigned w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round-to-nearest-even pack of two floats into one dword of bf16 (lo, hi);
// lowers to v_cvt_pk_bf16_f32 on gfx950.
SHRIMP_DEV unsigned pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  unsigned r = __builtin_bit_cast(unsigned, v);
  // opaque to the vectorisers: merged into wider vectors, the conversions are
  // split into one v_cvt_pk_bf16_f32 per value plus a v_perm_b32 per pair
  asm("" : "+v"(r));
  return r;
}

SHRIMP_DEV unsigned short f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(unsigned short, b);
}

SHRIMP_DEV float bf16_bits_to_f32(unsigned short h) {
  return __uint_as_float(((unsigned)h) << 16);
}

// Token rows of position b: seq[b, t, :] = bf16(tokens[t, :]) and, when tok_lo
// is given, tok_lo[b, t, :] = bf16(tokens[t, :] - that), by the workgroup's
// threads. vec4: four elements per thread and iteration (a 16-byte load, 8-byte
// stores); the host sets it when the element count is a multiple of 4 and the
// tables and rows are aligned for it. The same arithmetic per element.
SHRIMP_DEV void fill_token_rows(int b, const float* __restrict__ tokens, int n_tokens, int C,
                                unsigned short* __restrict__ seq, int64_t seq_sb,
                                unsigned short* __restrict__ tok_lo, int vec4) {
  const int n = n_tokens * C;
  if (vec4) {
    for (int i = 4 * (int)threadIdx.x; i < n; i += 4 * (int)blockDim.x) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(tokens + i);
      unsigned short hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = f32_to_bf16_bits(t[e]);
        lo[e] = f32_to_bf16_bits(t[e] - bf16_bits_to_f32(hi[e]));
      }
      *reinterpret_cast<u32x2*>(seq + (int64_t)b * seq_sb + i) =
          u32x2{hi[0] | ((unsigned)hi[1] << 16), hi[2] | ((unsigned)hi[3] << 16)};
      if (tok_lo)
        *reinterpret_cast<u32x2*>(tok_lo + (int64_t)b * n + i) =
            u32x2{lo[0] | ((unsigned)lo[1] << 16), lo[2] | ((unsigned)lo[3] << 16)};
    }
    return;
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float t = tokens[i];
    const unsigned short hi = f32_to_bf16_bits(t);
    seq[(int64_t)b * seq_sb + i] = hi;
    if (tok_lo) tok_lo[(int64_t)b * n + i] = f32_to_bf16_bits(t - bf16_bits_to_f32(hi));
  }
}

// ---- MFMA wrappers -------------------------------------------------------------

SHRIMP_DEV f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

SHRIMP_DEV f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// ---- cross-lane -----------------------------------------------------------------

// Index of this wave in its workgroup, as a wave-uniform (scalar) value: the
// compiler cannot prove threadIdx.x / 64 uniform, and loops bounded by a value
// it takes as divergent are built as masked loops whose memory requests it
// can no longer count precisely.
SHRIMP_DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

SHRIMP_DEV float xor_shfl(float v, int mask) { return __shfl_xor(v, mask, 64); }

// max(v, 0) as a signed integer max of the bit pattern: one instruction where
// fmaxf(v, 0) on a value the compiler cannot prove canonical (an MFMA result)
// takes two. Equal to fmaxf(v, 0) for every v except a NaN with the sign bit
// clear, which it passes through (fmaxf returns 0).
SHRIMP_DEV float relu_bits(float v) {
  return __builtin_bit_cast(float, max(__builtin_bit_cast(int, v), 0));
}

// Sum over the 4 lane groups (l/16 = 0..3) sharing the same l % 16.
SHRIMP_DEV float sum_lane_groups(float v) {
  v += xor_shfl(v, 16);
  v += xor_shfl(v, 32);
  return v;
}
SHRIMP_DEV float max_lane_groups(float v) {
  v = fmaxf(v, xor_shfl(v, 16));
  v = fmaxf(v, xor_shfl(v, 32));
  return v;
}

// Sum / max over the 4 lane groups on VALU lane swaps (v_permlane16_swap,
// v_permlane32_swap) instead of LDS-routed shuffles. Every lane of a group
// gets the bit-identical result (the pair sums are commutative).
SHRIMP_DEV float sum_groups_swap(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
SHRIMP_DEV float max_groups_swap(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sum over aligned groups of G lanes (G = 2, 4, 8, 16) with DPP lane moves on
// the VALU instead of LDS-routed shuffles, the same bits as the butterfly
// v += shfl_xor(v, m) for m = 1, 2, 4, 8: after the steps within a quad every
// lane of the quad holds the same value, so the mirror moves (lane i <- 7 - i
// in each half row, then i <- 15 - i in the row) bring the partner quad's or
// half's value as the xor 4 and xor 8 partners would (addition commutes).
template <int G>
SHRIMP_DEV float group_sum_dpp(float v) {
  static_assert(G == 2 || G == 4 || G == 8 || G == 16, "group of 2 to 16 lanes");
#define SHRIMP_DPP_MOV(x, ctrl) \
  __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ctrl, 0xF, 0xF, false))
  v += SHRIMP_DPP_MOV(v, 0xB1);                        // quad_perm [1, 0, 3, 2]: xor 1
  if constexpr (G >= 4) v += SHRIMP_DPP_MOV(v, 0x4E);   // quad_perm [2, 3, 0, 1]: xor 2
  if constexpr (G >= 8) v += SHRIMP_DPP_MOV(v, 0x141);  // row_half_mirror
  if constexpr (G >= 16) v += SHRIMP_DPP_MOV(v, 0x140); // row_mirror
#undef SHRIMP_DPP_MOV
  return v;
}

// ---- LayerNorm of 16 rows of 128 channels, MFMA operand layout ------------------
//
// Lane (lr, lg) holds channels 32 ks + 8 lg + e (ks < 4, e < 8) of row lr in
// xf[ks] (bf16); hf receives the normalised row without affine, bf16, in the
// same layout (the B operand of a 16x16x32 MFMA against output-major weight
// fragments, or its A operand against input-major ones). Statistics are fp32:
// mean first, then the centred sum of squares. An all-zero row gives zeros.
SHRIMP_DEV void ln_row128(const u32x4 (&xf)[4], float eps, u32x4 (&hf)[4]) {
  float s = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int w = 0; w < 4; ++w) s += bf16_lo(xf[ks][w]) + bf16_hi(xf[ks][w]);
  const float mean = sum_groups_swap(s) * (1.0f / 128);
  float q = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float u0 = bf16_lo(xf[ks][w]) - mean, u1 = bf16_hi(xf[ks][w]) - mean;
      q = fmaf(u0, u0, fmaf(u1, u1, q));
    }
  const float rstd = rsqrtf(sum_groups_swap(q) * (1.0f / 128) + eps);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int w = 0; w < 4; ++w)
      hf[ks][w] = pack_bf16x2((bf16_lo(xf[ks][w]) - mean) * rstd, (bf16_hi(xf[ks][w]) - mean) * rstd);
}

// ---- packed LN1 + q/k/v weights of the attention block (C = 128) -----------------
//
// shrimp_pack_attn_qkv output: bf16 MFMA fragments of W' = Wqkv diag(ln1_w)
// (rows: q 0-127, k 128-255, v 256-383), fragment (ks, nb) holding outputs
// 16 nb .. +15 over input channels 32 ks .. +31, lane (lr, lg) at byte
// ((ks * 24 + nb) * 64 + lane) * 16 with output 16 nb + lr and inputs
// 32 ks + 8 lg .. +7; then the 384 folded fp32 biases b' = bqkv + Wqkv ln1_b;
// then the 384 fp32 column sums cs[n] = sum_k W'[n][k] of the bf16 weights
// (LN(x) W'^T = rstd (x W'^T - mean cs) lets a kernel feed raw rows to MFMA).
constexpr int QKV_C = 128;
constexpr int QKV_N = 3 * QKV_C;
constexpr int QKV_NB = QKV_N / 16;
constexpr uint32_t QKV_W_BYTES = QKV_C * QKV_N * 2;
constexpr uint32_t QKV_B_OFF = QKV_W_BYTES;
constexpr uint32_t QKV_CS_OFF = QKV_B_OFF + QKV_N * 4;  // fp32 sum over k of the bf16 W'[n][k]
constexpr uint32_t QKV_PACK_BYTES = QKV_CS_OFF + QKV_N * 4;

// ---- per-channel biases held in registers -------------------------------------
//
// NT blocks of 16 channels kept in NT / 4 registers. A 16x16 accumulator
// fragment with rows = channels wants, at lane (lr, lg), channels
// 16 t + 4 lg + j (j = 0..3) of block t, the same four values across each
// 16-lane row lg. Register r therefore holds at lane (lr, lg) channel
// 16 (4 r + lr / 4) + 4 lg + lr % 4: row lg keeps exactly the values its
// lanes need, and rows(t) takes them with four DPP row broadcasts
// (row_newbcast of lane 4 (t % 4) + j of register t / 4): exact copies, four
// VALU moves per block. This keeps bias loads out of loops whose global loads
// would otherwise make each bias wait for every earlier load and store
// (memory operations retire in order).
template <int NT>
struct BiasRegs {
  static_assert(NT % 4 == 0, "bias blocks come in fours");
  float reg[NT / 4];

  SHRIMP_DEV void load(const float* bias, int lane) {
    const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int r = 0; r < NT / 4; ++r) reg[r] = bias[16 * (4 * r + lr / 4) + 4 * lg + lr % 4];
  }
  // 16x16 fragment with rows = channels: lane (lr, lg) gets bias[16 t + 4 lg + j]
  // (t is a constant once the caller's loops are unrolled)
  SHRIMP_DEV f32x4 rows(int t) const {
    const int v = __builtin_bit_cast(int, reg[t >> 2]);
    switch (t & 3) {
      case 0: return bcast4<0>(v);
      case 1: return bcast4<4>(v);
      case 2: return bcast4<8>(v);
      default: return bcast4<12>(v);
    }
  }

 private:
  // lanes S .. S + 3 of each 16-lane row, broadcast over the row
  // (row_newbcast with every row and bank enabled writes every lane, so no
  // old value is needed: update_dpp with an old value of 0 costs a v_mov of
  // 0 per broadcast)
  template <int S>
  SHRIMP_DEV static f32x4 bcast4(int v) {
    return f32x4{
        __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x150 + S, 0xF, 0xF, false)),
        __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x151 + S, 0xF, 0xF, false)),
        __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x152 + S, 0xF, 0xF, false)),
        __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x153 + S, 0xF, 0xF, false))};
  }
};

SHRIMP_DEV float wave_sum(float v) {
  for (int m = 32; m >= 1; m >>= 1) v += xor_shfl(v, m);
  return v;
}

// erf-based GELU (torch.nn.functional.gelu default, approximate='none').
SHRIMP_DEV float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }
