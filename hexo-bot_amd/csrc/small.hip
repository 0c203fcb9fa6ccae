// Small per-position kernels around the Shrimp forward: input preparation,
// token rows, the trunk tail (final LayerNorm + pooled value head), serve
// decode, and the pair / ray index builders. One workgroup per position; all
// are bandwidth-trivial next to the conv and attention kernels.
#include "capi.hpp"
#include "common.hpp"

#include <mutex>

namespace shrimp {

// Typed loads for the flat preparation loops (the element type is chosen once,
// outside the loop, so the loop body has no branch and keeps loads in flight).
template <int DT>
SHRIMP_DEV int64_t load_index_t(const void* __restrict__ p, int64_t i) {
  if constexpr (DT == SHRIMP_DT_I64) return static_cast<const int64_t*>(p)[i];
  else if constexpr (DT == SHRIMP_DT_I32) return static_cast<const int32_t*>(p)[i];
  else {
    const unsigned v = static_cast<const uint16_t*>(p)[i];
    return v == 0xFFFFu ? -1 : (int64_t)v;
  }
}
template <int DT>
SHRIMP_DEV float load_feat_t(const void* __restrict__ p, int64_t i) {
  if constexpr (DT == SHRIMP_DT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == SHRIMP_DT_F16) return (float)static_cast<const _Float16*>(p)[i];
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// idx rows of one position: tap 0 = the cell itself, taps 1..6 its neighbours
// (outside [0, N) -> N).
// Each loop runs over the elements i0, i0 + step, ... of one position.
template <int DT>
SHRIMP_DEV void prep_idx(const void* __restrict__ nbr, int64_t base, int N, int32_t* __restrict__ ib,
                         int i0, int step) {
#pragma unroll 4
  for (int i = i0; i < N * 7; i += step) {
    const int n = i / 7, k = i - n * 7;
    int32_t v = n;
    if (k > 0) {
      const int64_t j = load_index_t<DT>(nbr, (base + n) * 6 + k - 1);
      SHRIMP_DCHECK((j >= -1 && j <= N) || (DT == SHRIMP_DT_U16 && j == 0xFFFF), SHRIMP_DBG_NBR);
      v = (j >= 0 && j < N) ? (int32_t)j : N;
    }
    ib[i] = v;
  }
}
// 16 dwords (32 bf16 channels) per cell, zero past nfeat.
template <int DT>
SHRIMP_DEV void prep_feats(const void* __restrict__ feats, int nfeat, int64_t base, int N,
                           unsigned* __restrict__ xb, int i0, int step) {
#pragma unroll 4
  for (int i = i0; i < N * 16; i += step) {
    const int f = (i & 15) * 2;
    const int64_t r = base + (i >> 4);
    const float v0 = f < nfeat ? load_feat_t<DT>(feats, r * nfeat + f) : 0.f;
    const float v1 = f + 1 < nfeat ? load_feat_t<DT>(feats, r * nfeat + f + 1) : 0.f;
    xb[i] = pack_bf16x2(v0, v1);
  }
}
// Mask, coords, seq_mask and seq_lens of one position: each thread loads a
// cell's mask byte and coordinates together (CDT: the coords dtype, 0 when
// coords32 is not wanted) and keeps 1 + the index of its last live cell.
template <int CDT>
SHRIMP_DEV int prep_cells(const uint8_t* __restrict__ mask, const void* __restrict__ coords,
                          int64_t base, int64_t sbase, int N, int n_tokens,
                          uint8_t* __restrict__ mask8, int32_t* __restrict__ c32,
                          uint8_t* __restrict__ seq_mask) {
  int last = 0;
#pragma unroll 2
  for (int n = threadIdx.x; n < N; n += blockDim.x) {
    const int64_t r = base + n;
    const bool live = mask[r] != 0;
    if constexpr (CDT != 0) {
      const int32_t c0 = (int32_t)load_index_t<CDT>(coords, r * 2);
      const int32_t c1 = (int32_t)load_index_t<CDT>(coords, r * 2 + 1);
      c32[r * 2] = c0;
      c32[r * 2 + 1] = c1;
    }
    if (mask8) mask8[r] = live ? 1 : 0;
    if (seq_mask) seq_mask[sbase + n_tokens + n] = live ? 1 : 0;
    if (live) last = n + 1;
  }
  return last;
}

// A position's outputs are written by PREP_PARTS workgroups (blockIdx.y), each
// with one kind of output, so a thread issues a single round of loads before
// its stores: parts [0, PREP_FEAT) the stem input rows, the next PREP_IDX the
// idx rows, the last one the mask, coords, seq_mask and seq_lens.
constexpr int PREP_FEAT = 4, PREP_IDX = 2, PREP_PARTS = PREP_FEAT + PREP_IDX + 1;
// prep_csr_kernel spreads its flat loops over PREP_CSR_PARTS workgroups per row
constexpr int PREP_CSR_PARTS = 4;

// ---- input preparation (model.py:861-863, 884-892; batching.py:264-276) --------
// Each output array is written by a flat loop over its elements, so
// consecutive lanes touch consecutive addresses. The pointers are __restrict__
// and the loops unrolled, so each thread keeps its loads in flight together
// instead of one load / wait / store per element.
__global__ __launch_bounds__(256) void prep_kernel(const void* __restrict__ nbr, int nbr_dt,
                                                   const void* __restrict__ mask,
                                                   const void* __restrict__ coords, int coords_dt,
                                                   const void* __restrict__ feats, int feats_dt,
                                                   int nfeat, int N, int n_tokens,
                                                   int32_t* __restrict__ idx,
                                                   uint8_t* __restrict__ mask8,
                                                   int32_t* __restrict__ coords32,
                                                   int32_t* __restrict__ seq_lens,
                                                   uint8_t* __restrict__ seq_mask,
                                                   uint16_t* __restrict__ xin) {
  const int b = blockIdx.x;
  const int part = blockIdx.y;  // uniform over the workgroup
  const int64_t base = (int64_t)b * N;
  if (part < PREP_FEAT) {
    if (!xin) return;
    const int i0 = part * blockDim.x + threadIdx.x, step = PREP_FEAT * blockDim.x;
    unsigned* xb = reinterpret_cast<unsigned*>(xin + base * 32);
    if (feats_dt == SHRIMP_DT_F32) prep_feats<SHRIMP_DT_F32>(feats, nfeat, base, N, xb, i0, step);
    else if (feats_dt == SHRIMP_DT_F16) prep_feats<SHRIMP_DT_F16>(feats, nfeat, base, N, xb, i0, step);
    else prep_feats<SHRIMP_DT_BF16>(feats, nfeat, base, N, xb, i0, step);
    return;
  }
  if (part < PREP_FEAT + PREP_IDX) {
    if (!idx) return;
    const int i0 = (part - PREP_FEAT) * blockDim.x + threadIdx.x, step = PREP_IDX * blockDim.x;
    int32_t* ib = idx + base * 7;
    if (nbr_dt == SHRIMP_DT_I64) prep_idx<SHRIMP_DT_I64>(nbr, base, N, ib, i0, step);
    else if (nbr_dt == SHRIMP_DT_I32) prep_idx<SHRIMP_DT_I32>(nbr, base, N, ib, i0, step);
    else prep_idx<SHRIMP_DT_U16>(nbr, base, N, ib, i0, step);
    return;
  }
  const uint8_t* m = static_cast<const uint8_t*>(mask);
  const int64_t sbase = (int64_t)b * (n_tokens + N);
  int last;
  if (!coords32) last = prep_cells<0>(m, coords, base, sbase, N, n_tokens, mask8, coords32, seq_mask);
  else if (coords_dt == SHRIMP_DT_I64)
    last = prep_cells<SHRIMP_DT_I64>(m, coords, base, sbase, N, n_tokens, mask8, coords32, seq_mask);
  else last = prep_cells<SHRIMP_DT_I32>(m, coords, base, sbase, N, n_tokens, mask8, coords32, seq_mask);
  if (seq_mask)
    for (int t = threadIdx.x; t < n_tokens; t += blockDim.x) seq_mask[sbase + t] = 1;
  if (seq_lens) {
    __shared__ int red[256];
    red[threadIdx.x] = last;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + s]);
      __syncthreads();
    }
    if (threadIdx.x == 0) seq_lens[b] = n_tokens + red[0];
  }
}

// Serve pack + index preparation from the ABI-1 payload arrays, one workgroup
// per row: row row0 + b occupies cells [off, off + n) of the CSR arrays, its
// live cells are the first n of the N padded ones. Same outputs and rules as
// prep_kernel on the host-packed batch (the 0xFFFF sentinel and indices >= N
// become N; padding rows are self-only, masked, zero).
__global__ __launch_bounds__(256) void prep_csr_kernel(const uint16_t* __restrict__ feats, int nfeat,
                                                       const int16_t* __restrict__ qr,
                                                       const uint16_t* __restrict__ nbr,
                                                       const int64_t* __restrict__ offsets, int row0,
                                                       int N, int n_tokens, int32_t* __restrict__ idx,
                                                       uint8_t* __restrict__ mask8,
                                                       int32_t* __restrict__ coords32,
                                                       int32_t* __restrict__ seq_lens,
                                                       uint8_t* __restrict__ seq_mask,
                                                       uint16_t* __restrict__ xin) {
  const int b = blockIdx.x;
  const int64_t o = offsets[row0 + b];
  const int64_t cnt = offsets[row0 + b + 1] - o;
  const int n = cnt < 0 ? 0 : (cnt > N ? N : (int)cnt);
  const int64_t base = (int64_t)b * N;
  const int i0 = blockIdx.y * blockDim.x + threadIdx.x;
  const int step = PREP_CSR_PARTS * blockDim.x;
  if (seq_mask && blockIdx.y == 0)
    for (int t = threadIdx.x; t < n_tokens; t += blockDim.x)
      seq_mask[(int64_t)b * (n_tokens + N) + t] = 1;
  // flat loops over each output array (consecutive lanes, consecutive addresses)
  if (idx) {
    int32_t* ib = idx + base * 7;
#pragma unroll 4
    for (int i = i0; i < N * 7; i += step) {
      const int r = i / 7, k = i - r * 7;
      int32_t v = r;
      if (k > 0) {
        const unsigned j = r < n ? nbr[(o + r) * 6 + k - 1] : 0xFFFFu;
        SHRIMP_DCHECK(j == 0xFFFFu || (int)j < n, SHRIMP_DBG_NBR);
        v = (int)j < N ? (int32_t)j : N;
      }
      ib[i] = v;
    }
  }
  if (xin) {
    unsigned* xb = reinterpret_cast<unsigned*>(xin + base * 32);
#pragma unroll 4
    for (int i = i0; i < N * 16; i += step) {
      const int r = i >> 4, f = (i & 15) * 2;
      const bool live = r < n;
      const int64_t c = o + r;
      const float v0 = live && f < nfeat ? (float)__builtin_bit_cast(_Float16, feats[c * nfeat + f]) : 0.f;
      const float v1 =
          live && f + 1 < nfeat ? (float)__builtin_bit_cast(_Float16, feats[c * nfeat + f + 1]) : 0.f;
      xb[i] = pack_bf16x2(v0, v1);
    }
  }
  if (coords32)
    for (int i = i0; i < N * 2; i += step)
      coords32[base * 2 + i] = (i >> 1) < n ? qr[o * 2 + i] : 0;
  for (int i = i0; i < N; i += step) {
    const int64_t r = base + i;
    const bool live = i < n;
    if (mask8) mask8[r] = live ? 1 : 0;
    if (seq_mask) seq_mask[(int64_t)b * (n_tokens + N) + n_tokens + i] = live ? 1 : 0;
  }
  if (seq_lens && blockIdx.y == 0 && threadIdx.x == 0) seq_lens[b] = n_tokens + n;
}

__global__ void fill_tokens_kernel(const float* __restrict__ tokens, int n_tokens, int C,
                                   uint16_t* __restrict__ seq, int64_t seq_sb,
                                   uint16_t* __restrict__ tok_lo, int vec4) {
  fill_token_rows(blockIdx.x, tokens, n_tokens, C, seq, seq_sb, tok_lo, vec4);
}

// ---- trunk tail + value heads (model.py:927-935, 990-1002) --------------------
// Sum over the TPR lanes of a row: DPP moves up to 16 lanes, then one shuffle
// (the butterfly order of v += shfl_xor(v, m), m = 1, 2, 4, ...).
template <int TPR>
SHRIMP_DEV float row_group_sum(float v) {
  if constexpr (TPR <= 16) {
    return group_sum_dpp<TPR>(v);
  } else {
    v = group_sum_dpp<16>(v);
#pragma unroll
    for (int m = 16; m < TPR; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
  }
}

// Pass 1, one workgroup per position: final LayerNorm of every row (cells
// masked), written to out_seq; the value-head inputs [T0 | T1 | pooled] and
// [T4 | T5 | pooled] go to the workspace (B, 6C) fp32.
// A row is handled by TPR = C / 8 lanes (8 channels each), 256 / TPR rows per
// pass, U passes per chunk, a chunk's rows and mask bytes requested at once
// (at C = 128 a position of up to 272 rows is one chunk). Rows go in and out
// through buffer resources (rows past S or channels past C at an offset past
// them), with no request or store under a branch. Row statistics reduce over
// the TPR lanes.
// F32: seq and out_seq hold fp32 rows instead of bf16 (the fp32 serve mode).
template <int TPR, bool F32>
__global__ __launch_bounds__(256) void final_ln_kernel(const shrimp_tail_args a, uint32_t seq_bytes,
                                                       uint32_t mask_bytes, uint32_t ws_bytes,
                                                       uint32_t lo_bytes) {
  constexpr int RPP = 256 / TPR;  // rows per pass
  constexpr int U = F32 ? 4 : 17;  // passes per chunk (bf16, C = 128: a position of up to 272 rows)
  constexpr int EB = F32 ? 4 : 2;  // bytes per element
  extern __shared__ float fl[];   // [RPP][C] pooled partial sums, then [RPP] counts
  const int b = blockIdx.x;
  const int C = a.C, S = a.S, nt = a.n_tokens, N = S - nt;
  const int t = threadIdx.x;
  const int sub = t % TPR;         // 8-channel chunk of this lane
  const int rs = t / TPR;          // row slot
  const int c0 = sub * 8;
  const bool cv = c0 < C;
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.seq, seq_bytes);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out_seq, seq_bytes);
  const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.mask, mask_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.workspace, ws_bytes);
  // token rows' low parts (lo_bytes 0 without them: reads give zeros); the
  // tokens are rows 0 .. nt - 1, all in the first pass (nt <= RPP)
  const __amdgpu_buffer_rsrc_t lr = make_rsrc(a.tok_lo, lo_bytes);
  const uint32_t pos_off = (uint32_t)((int64_t)b * a.s_sb * EB);
  const uint32_t vin_off = (uint32_t)((int64_t)b * 6 * C * 4);
  float w[8], bb[8], pool[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = cv ? a.ln_w[c0 + e] : 0.f;
    bb[e] = cv ? a.ln_b[c0 + e] : 0.f;
    pool[e] = 0.f;
  }
  int cnt = 0;
  const float invc = 1.0f / (float)C;
  const int nchunk = (S + U * RPP - 1) / (U * RPP);
  // byte offset of this lane's 8 channels of row `row`, or past the buffer
  auto row_off = [&](int row) {
    return row < S && cv ? pos_off + (uint32_t)((row * C + c0) * EB) : SHRIMP_OOB_OFFSET;
  };
  constexpr int U2 = F32 ? U : 1;  // second 16 bytes of an fp32 row chunk
  auto load = [&](int chunk, u32x4 (&raw)[U], u32x4 (&raw2)[U2], unsigned (&mk)[U], u32x4& lo0) {
    lo0 = buf_load16(lr, chunk == 0 && rs < nt && cv
                             ? (uint32_t)((((int64_t)b * nt + rs) * C + c0) * 2)
                             : SHRIMP_OOB_OFFSET);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = chunk * U * RPP + u * RPP + rs;
      const uint32_t off = chunk < nchunk ? row_off(row) : SHRIMP_OOB_OFFSET;
      raw[u] = buf_load16(sr, off);
      if constexpr (F32) raw2[u] = buf_load16(sr, off + 16);
      const bool cell = row >= nt && row < S && chunk < nchunk;
      mk[u] = (unsigned)__builtin_amdgcn_raw_buffer_load_b8(
          mr, cell ? (uint32_t)((int64_t)b * N + (row - nt)) : SHRIMP_OOB_OFFSET, 0, 0);
    }
  };
  for (int ch = 0; ch < nchunk; ++ch) {
    u32x4 raw[U], raw2[U2], lo0;
    unsigned mk[U];
    load(ch, raw, raw2, mk, lo0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = ch * U * RPP + u * RPP + rs;
      float x[8];
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (F32) {
          x[e] = __uint_as_float(raw[u][e]);
          x[4 + e] = __uint_as_float(raw2[u][e]);
        } else if (u == 0) {
          x[2 * e] = bf16_lo(raw[u][e]) + bf16_lo(lo0[e]);
          x[2 * e + 1] = bf16_hi(raw[u][e]) + bf16_hi(lo0[e]);
        } else {
          x[2 * e] = bf16_lo(raw[u][e]);
          x[2 * e + 1] = bf16_hi(raw[u][e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) s += x[e];
      s = row_group_sum<TPR>(s);
      const float mean = s * invc;
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = cv ? x[e] - mean : 0.f;
        q = fmaf(x[e], x[e], q);
      }
      q = row_group_sum<TPR>(q);
      const float rstd = rsqrtf(q * invc + a.eps);
      const bool rv = row < S && cv;
      const bool cell = row >= nt;
      const bool live = !cell || mk[u] != 0;
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = live ? fmaf(x[e] * rstd, w[e], bb[e]) : 0.f;
      const uint32_t off = row_off(row);
      if constexpr (F32) {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3])},
            orr, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]), __float_as_uint(y[7])},
            orr, off + 16, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                  pack_bf16x2(y[6], y[7])},
            orr, off, 0, 0);
      }
      // pooled cells (dead ones add zeros); token rows 0, 1 feed the value
      // head, rows 4, 5 the moves-left head
      const bool pooled = rv && cell;
      if (pooled && live && sub == 0) ++cnt;
#pragma unroll
      for (int e = 0; e < 8; ++e) pool[e] += pooled ? y[e] : 0.f;
      const int slot = row == 0 ? 0 : row == 1 ? 1 : row == 4 ? 3 : row == 5 ? 4 : -1;
      const uint32_t voff = rv && slot >= 0 ? vin_off + (uint32_t)((slot * C + c0) * 4) : SHRIMP_OOB_OFFSET;
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3])},
          wr, voff, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]), __float_as_uint(y[7])},
          wr, voff + 16, 0, 0);
    }
  }
  float* vin = a.workspace + (int64_t)b * 6 * C;
  float* red = fl;                 // [RPP][C]
  float* cred = fl + RPP * C;      // [RPP]
  if (cv) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[rs * C + c0 + e] = pool[e];
  }
  if (sub == 0) cred[rs] = (float)cnt;
  __syncthreads();
  float total = 0.f;
  for (int i = 0; i < RPP; ++i) total += cred[i];
  const float inv = 1.0f / fmaxf(1.f, total);
  for (int c = t; c < C; c += blockDim.x) {
    float p = 0.f;
    for (int i = 0; i < RPP; ++i) p += red[i * C + c];
    vin[2 * C + c] = p * inv;
    vin[5 * C + c] = p * inv;
  }
}

// Pass 2: one head (value or moves-left, blockIdx.y) for kHeadPos positions
// per workgroup: hid = relu(in @ Wr + br) (in = [T | T' | pooled], 3C),
// out = hid @ Wh + bh. Weights are transposed (k-major) so consecutive lanes read consecutive
// outputs; the K range is split over the kHeadThreads / C (then / bins)
// thread slices and reduced through LDS.
constexpr int kHeadPos = 4;
constexpr int kHeadThreads = 1024;
__global__ __launch_bounds__(kHeadThreads) void value_head_kernel(const shrimp_tail_args a) {
  extern __shared__ float hs[];
  const int C = a.C, bins = a.bins, K1 = 3 * C;
  const int head = blockIdx.y;
  const float* rwt = head == 0 ? a.vr_w : a.mr_w;
  const float* rb = head == 0 ? a.vr_b : a.mr_b;
  const float* hwt = head == 0 ? a.vh_w : a.mh_w;
  const float* hb = head == 0 ? a.vh_b : a.mh_b;
  float* dst = head == 0 ? a.value : a.moves_left;
  if (dst == nullptr) return;  // uniform
  const int b0 = blockIdx.x * kHeadPos;
  const int np = min(kHeadPos, a.B - b0);
  const int t = threadIdx.x;
  const int ks1 = kHeadThreads / C;     // K slices, layer 1
  const int ks2 = kHeadThreads / bins;  // K slices, layer 2
  float* in = hs;                              // [kHeadPos][K1]
  float* red = in + kHeadPos * K1;             // [ks1][kHeadPos][C]
  float* hid = red + ks1 * kHeadPos * C;       // [kHeadPos][C]
  float* red2 = hid + kHeadPos * C;            // [ks2][kHeadPos][bins]
  for (int i = t; i < kHeadPos * K1; i += blockDim.x) {
    const int p = i / K1, k = i - p * K1;
    in[i] = p < np ? a.workspace[(int64_t)(b0 + p) * 6 * C + head * K1 + k] : 0.f;
  }
  __syncthreads();
  {
    const int o = t % C, ks = t / C;
    if (ks < ks1) {
      const int k0 = ks * K1 / ks1, k1 = (ks + 1) * K1 / ks1;
      float s[kHeadPos] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = k0; k < k1; ++k) {
        const float w = rwt[(int64_t)k * C + o];
#pragma unroll
        for (int p = 0; p < kHeadPos; ++p) s[p] = fmaf(w, in[p * K1 + k], s[p]);
      }
#pragma unroll
      for (int p = 0; p < kHeadPos; ++p) red[(ks * kHeadPos + p) * C + o] = s[p];
    }
  }
  __syncthreads();
  for (int i = t; i < kHeadPos * C; i += blockDim.x) {
    const int p = i / C, o = i - p * C;
    float s = rb[o];
    for (int ks = 0; ks < ks1; ++ks) s += red[(ks * kHeadPos + p) * C + o];
    hid[i] = fmaxf(s, 0.f);
  }
  __syncthreads();
  {
    const int o = t % bins, ks = t / bins;
    if (ks < ks2) {
      const int k0 = ks * C / ks2, k1 = (ks + 1) * C / ks2;
      float s[kHeadPos] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = k0; k < k1; ++k) {
        const float w = hwt[(int64_t)k * bins + o];
#pragma unroll
        for (int p = 0; p < kHeadPos; ++p) s[p] = fmaf(w, hid[p * C + k], s[p]);
      }
#pragma unroll
      for (int p = 0; p < kHeadPos; ++p) red2[(ks * kHeadPos + p) * bins + o] = s[p];
    }
  }
  __syncthreads();
  for (int i = t; i < kHeadPos * bins; i += blockDim.x) {
    const int p = i / bins, o = i - p * bins;
    if (p >= np) continue;
    float s = hb[o];
    for (int ks = 0; ks < ks2; ++ks) s += red2[(ks * kHeadPos + p) * bins + o];
    dst[(int64_t)(b0 + p) * bins + o] = s;
  }
}

// ---- serve decode (inference.py:998-1042, losses.py:40-60) ---------------------
__device__ float block_reduce(float v, bool is_max, float* red) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  for (int m = 32; m >= 1; m >>= 1) {
    const float o = __shfl_xor(v, m, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__device__ float decode_expectation(const float* logits, int bins, float* red) {
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < bins; i += blockDim.x) mx = fmaxf(mx, logits[i]);
  mx = block_reduce(mx, true, red);
  float se = 0.f, sv = 0.f;
  const float step = 2.0f / (float)(bins - 1);
  for (int i = threadIdx.x; i < bins; i += blockDim.x) {
    const float e = expf(logits[i] - mx);
    const float bin = (2 * i < bins) ? -1.0f + step * i : 1.0f - step * (bins - 1 - i);
    se += e;
    sv += e * bin;
  }
  se = block_reduce(se, false, red);
  sv = block_reduce(sv, false, red);
  const float v = sv / se;
  return fminf(fmaxf(v, -1.0f), 1.0f);
}

__global__ __launch_bounds__(256) void decode_kernel(const float* value_logits,
                                                     const float* ml_logits, const float* policy,
                                                     int64_t pol_sb, const int32_t* legal,
                                                     const int64_t* out_off, int bins,
                                                     float ml_cap, float* value, float* ml,
                                                     float* priors, float* logits_out) {
  __shared__ float red[8];
  const int b = blockIdx.x;
  const float v = decode_expectation(value_logits + (int64_t)b * bins, bins, red);
  if (threadIdx.x == 0) value[b] = v;
  if (ml_logits != nullptr) {
    const float u = decode_expectation(ml_logits + (int64_t)b * bins, bins, red);
    if (threadIdx.x == 0) ml[b] = (u + 1.0f) * 0.5f * ml_cap;
  }
  // The legal prefix never extends past the row (pol_sb == Npad here).
  SHRIMP_DCHECK(legal[b] >= 0 && legal[b] <= pol_sb, SHRIMP_DBG_LEGAL);
  const int L = max(0, min(legal[b], (int)pol_sb));
  const float* row = policy + (int64_t)b * pol_sb;
  float* dst = priors + out_off[b];
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < L; i += blockDim.x) mx = fmaxf(mx, row[i]);
  mx = block_reduce(mx, true, red);
  float se = 0.f;
  for (int i = threadIdx.x; i < L; i += blockDim.x) se += expf(row[i] - mx);
  se = block_reduce(se, false, red);
  const float inv = 1.0f / se;
  for (int i = threadIdx.x; i < L; i += blockDim.x) {
    dst[i] = expf(row[i] - mx) * inv;
    if (logits_out != nullptr) logits_out[out_off[b] + i] = row[i];
  }
}

// ---- pair index (model.py:762-792) ------------------------------------------------
__global__ void pair_kernel(const int32_t* coords, const uint8_t* mask, const uint8_t* lut,
                            int M, int N, int nt, int r_ct, int r_tc, int r_tt, int pad_row,
                            uint8_t* pair) {
  const int b = blockIdx.y;
  const int i = blockIdx.x;  // query row
  const int S = nt + N;
  const int W = 2 * M + 1;
  for (int j = threadIdx.x; j < S; j += blockDim.x) {
    int row;
    const bool qt = i < nt, kt = j < nt;
    if (qt && kt) row = r_tt;
    else if (qt) row = r_tc;
    else if (kt) row = r_ct;
    else {
      const int64_t ci = (int64_t)b * N + (i - nt), cj = (int64_t)b * N + (j - nt);
      int dq = coords[cj * 2] - coords[ci * 2];
      int dr = coords[cj * 2 + 1] - coords[ci * 2 + 1];
      dq = dq < -M ? -M : (dq > M ? M : dq);
      dr = dr < -M ? -M : (dr > M ? M : dr);
      row = lut[(dq + M) * W + (dr + M)];
    }
    if (!kt && mask[(int64_t)b * N + (j - nt)] == 0) row = pad_row;
    pair[((int64_t)b * S + i) * S + j] = (uint8_t)row;
  }
}

// ---- ray gather index (hexfield_eq/_triton_ray.py:221-281) ------------------------
// Per position: an LDS open-addressing table of live cells keyed by packed
// (q, r), then one probe per (cell, slot). Coordinates must satisfy
// |q|, |r| < 2^14; cells outside that domain are never matched.
#define RAY_TABLE 4096
__device__ __forceinline__ unsigned ray_key(int q, int r) {
  if (q <= -16384 || q >= 16384 || r <= -16384 || r >= 16384) return 0u;
  return ((unsigned)(q + 16384) << 15 | (unsigned)(r + 16384)) + 1u;
}
__device__ __forceinline__ unsigned ray_hash(unsigned k) { return (k * 2654435761u) >> 20; }

__global__ __launch_bounds__(256) void ray_index_kernel(const int32_t* coords, const uint8_t* mask,
                                                        int N, int32_t* idx) {
  __shared__ unsigned keys[RAY_TABLE];
  __shared__ int vals[RAY_TABLE];
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < RAY_TABLE; i += blockDim.x) keys[i] = 0u;
  __syncthreads();
  for (int n = threadIdx.x; n < N; n += blockDim.x) {
    const int64_t r = (int64_t)b * N + n;
    if (!mask[r]) continue;
    const unsigned k = ray_key(coords[r * 2], coords[r * 2 + 1]);
    if (k == 0u) continue;
    unsigned h = ray_hash(k) & (RAY_TABLE - 1);
    for (int probe = 0; probe < RAY_TABLE; ++probe) {
      const unsigned prev = atomicCAS(&keys[h], 0u, k);
      if (prev == 0u || prev == k) {
        vals[h] = n;
        break;
      }
      h = (h + 1) & (RAY_TABLE - 1);
    }
  }
  __syncthreads();
  const int ax_q[3] = {1, 0, 1}, ax_r[3] = {0, 1, -1};
  for (int i = threadIdx.x; i < N * 32; i += blockDim.x) {
    const int n = i >> 5;
    const int s = i & 31;
    const int64_t r = (int64_t)b * N + n;
    int out = N;
    if (s == 0) {
      out = n;
    } else if (s < 31) {
      const int t = s - 1;
      const int axis = t / 10, dir = (t % 10) / 5, k = t % 5 + 1;
      const int sgn = dir == 0 ? 1 : -1;
      const unsigned key =
          ray_key(coords[r * 2] + sgn * k * ax_q[axis], coords[r * 2 + 1] + sgn * k * ax_r[axis]);
      if (key != 0u) {
        unsigned h = ray_hash(key) & (RAY_TABLE - 1);
        for (int probe = 0; probe < RAY_TABLE; ++probe) {
          const unsigned kk = keys[h];
          if (kk == key) {
            out = vals[h];
            break;
          }
          if (kk == 0u) break;
          h = (h + 1) & (RAY_TABLE - 1);
        }
      }
    }
    idx[r * 32 + s] = out;
  }
}

}  // namespace shrimp

using namespace shrimp;

extern "C" int shrimp_prep_inputs(const void* nbr, int nbr_dt, const void* mask, const void* coords,
                                  int coords_dt, const void* feats, int feats_dt, int nfeat, int B,
                                  int N, int n_tokens, int32_t* idx, uint8_t* mask8,
                                  int32_t* coords32, int32_t* seq_lens, uint8_t* seq_mask,
                                  void* xin, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && N > 0 && N <= kMaxDim, "prep_inputs: bad shape (%d, %d)", B, N);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(mask != nullptr, "prep_inputs: mask required");
  SHRIMP_REQUIRE(n_tokens >= 0 && n_tokens <= 4096, "prep_inputs: n_tokens %d", n_tokens);
  SHRIMP_REQUIRE(!idx || (nbr && (nbr_dt == SHRIMP_DT_I64 || nbr_dt == SHRIMP_DT_I32 ||
                                  nbr_dt == SHRIMP_DT_U16)),
                 "prep_inputs: nbr dtype");
  SHRIMP_REQUIRE(!coords32 || (coords && (coords_dt == SHRIMP_DT_I64 || coords_dt == SHRIMP_DT_I32)),
                 "prep_inputs: coords dtype");
  SHRIMP_REQUIRE(!xin || (feats && nfeat > 0 && nfeat <= 32 &&
                          (feats_dt == SHRIMP_DT_F32 || feats_dt == SHRIMP_DT_F16 ||
                           feats_dt == SHRIMP_DT_BF16)),
                 "prep_inputs: feats dtype / width");
  hipLaunchKernelGGL(prep_kernel, dim3(B, PREP_PARTS), dim3(256), 0, as_stream(stream), nbr, nbr_dt, mask,
                     coords, coords_dt, feats, feats_dt, nfeat, N, n_tokens, idx, mask8, coords32,
                     seq_lens, seq_mask, static_cast<uint16_t*>(xin));
  return check_launch("prep_inputs");
}

extern "C" int shrimp_prep_csr(const void* node_feats, int nfeat, const int16_t* node_qr,
                               const uint16_t* nbr, const int64_t* row_offsets, int row0, int B,
                               int N, int n_tokens, int32_t* idx, uint8_t* mask8, int32_t* coords32,
                               int32_t* seq_lens, uint8_t* seq_mask, void* xin, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && N > 0 && N <= kMaxDim && row0 >= 0 && n_tokens >= 0 && n_tokens <= 4096,
                 "prep_csr: bad sizes");
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(row_offsets, "prep_csr: null row offsets");
  SHRIMP_REQUIRE(!idx || nbr, "prep_csr: idx needs nbr");
  SHRIMP_REQUIRE(!coords32 || node_qr, "prep_csr: coords need node_qr");
  SHRIMP_REQUIRE(!xin || (node_feats && nfeat > 0 && nfeat <= 32), "prep_csr: feats (nfeat %d)",
                 nfeat);
  hipLaunchKernelGGL(prep_csr_kernel, dim3(B, PREP_CSR_PARTS), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(node_feats), nfeat, node_qr, nbr, row_offsets,
                     row0, N, n_tokens, idx, mask8, coords32, seq_lens, seq_mask,
                     static_cast<uint16_t*>(xin));
  return check_launch("prep_csr");
}

// Checks the token-row arguments and returns the vec4 switch of
// fill_token_rows (0 or 1), or SHRIMP_EINVAL with the error set. With no rows
// to write (B or n_tokens 0) only the sizes are checked.
int shrimp::fill_tokens_check(const float* tokens, int n_tokens, int C, const void* seq,
                              int64_t seq_sb, const void* tok_lo, int B) {
  SHRIMP_REQUIRE(B >= 0 && n_tokens >= 0 && n_tokens <= 4096 && C > 0 && C <= 4096,
                 "fill_tokens: bad sizes (B %d, tokens %d, C %d)", B, n_tokens, C);
  if (B == 0 || n_tokens == 0) return 0;
  SHRIMP_REQUIRE(tokens && seq, "fill_tokens: null pointer");
  SHRIMP_REQUIRE(strides_ok({seq_sb}) && seq_sb >= (int64_t)n_tokens * C,
                 "fill_tokens: position stride %lld", (long long)seq_sb);
  const int n = n_tokens * C;
  return n % 4 == 0 && seq_sb % 4 == 0 && (uintptr_t)tokens % 16 == 0 &&
         (uintptr_t)seq % 8 == 0 && (uintptr_t)tok_lo % 8 == 0;
}

extern "C" int shrimp_fill_tokens(const float* tokens, int n_tokens, int C, void* seq,
                                  int64_t seq_sb, void* tok_lo, int B, void* stream) {
  const int vec4 = fill_tokens_check(tokens, n_tokens, C, seq, seq_sb, tok_lo, B);
  if (vec4 < 0) return vec4;
  if (B == 0 || n_tokens == 0) return SHRIMP_OK;
  hipLaunchKernelGGL(fill_tokens_kernel, dim3(B), dim3(256), 0, as_stream(stream), tokens,
                     n_tokens, C, static_cast<uint16_t*>(seq), seq_sb,
                     static_cast<uint16_t*>(tok_lo), vec4);
  return check_launch("fill_tokens");
}

// Checks the tail arguments (all but the workspace) and launches the two
// passes with the head inputs in `ws` ((B, 6C) fp32, device memory).
static int launch_trunk_tail(const shrimp_tail_args* a, float* ws, hipStream_t st,
                             bool f32 = false) {
  SHRIMP_REQUIRE(a->B > 0 && a->S > 0 && a->S <= kMaxDim, "trunk_tail: bad shape (B %d, S %d)", a->B,
                 a->S);
  SHRIMP_REQUIRE(a->seq && a->mask && a->ln_w && a->ln_b && a->out_seq,
                 "trunk_tail: null pointer");
  SHRIMP_REQUIRE(a->C > 0 && a->C <= 256 && a->C % 2 == 0, "trunk_tail: C %d outside (0, 256]",
                 a->C);
  SHRIMP_REQUIRE(strides_ok({a->s_sb}) && a->s_sb % 2 == 0, "trunk_tail: position stride must be even");
  SHRIMP_REQUIRE(a->n_tokens >= 6 && a->S > a->n_tokens, "trunk_tail: needs >= 6 tokens");
  SHRIMP_REQUIRE(!a->value || (a->vr_w && a->vr_b && a->vh_w && a->vh_b), "trunk_tail: value head");
  SHRIMP_REQUIRE(!a->moves_left || (a->mr_w && a->mr_b && a->mh_w && a->mh_b),
                 "trunk_tail: moves-left head");
  SHRIMP_REQUIRE(a->C % 8 == 0 && a->C <= 256 && a->s_sb % 8 == 0,
                 "trunk_tail: C %d must be a multiple of 8 (<= 256), position stride of 8", a->C);
  SHRIMP_REQUIRE(a->bins > 0 && a->bins <= 256, "trunk_tail: bins %d", a->bins);
  SHRIMP_REQUIRE(!a->tok_lo || !f32, "trunk_tail_f32: token low parts apply to the bf16 stream only");
  SHRIMP_REQUIRE(a->n_tokens <= 8 * (256 / a->C), "trunk_tail: %d tokens exceed one pass of rows",
                 a->n_tokens);
  shrimp_tail_args k = *a;
  k.workspace = ws;
  const int64_t seq_bytes = ((int64_t)(k.B - 1) * k.s_sb + (int64_t)k.S * k.C) * (f32 ? 4 : 2);
  const int64_t mask_bytes = (int64_t)k.B * (k.S - k.n_tokens);
  const int64_t ws_bytes = (int64_t)k.B * 6 * k.C * 4;
  const int64_t lo_bytes = k.tok_lo ? (int64_t)k.B * k.n_tokens * k.C * 2 : 0;
  SHRIMP_REQUIRE(seq_bytes < (int64_t)0x7FFF0000 && ws_bytes < (int64_t)0x7FFF0000,
                 "trunk_tail: buffers too large for 32-bit offsets");
  const int tpr = k.C / 8;
  const size_t lsm = (size_t)(256 / ((tpr <= 4) ? 4 : (tpr <= 8) ? 8 : (tpr <= 16) ? 16 : 32)) *
                     (k.C + 1) * sizeof(float);
#define SHRIMP_FLN(T)                                                                      \
  do {                                                                                       \
    if (f32)                                                                                 \
      hipLaunchKernelGGL((final_ln_kernel<T, true>), dim3(k.B), dim3(256), lsm, st, k,         \
                         (uint32_t)seq_bytes, (uint32_t)mask_bytes, (uint32_t)ws_bytes,        \
                         (uint32_t)lo_bytes);                                                  \
    else                                                                                     \
      hipLaunchKernelGGL((final_ln_kernel<T, false>), dim3(k.B), dim3(256), lsm, st, k,        \
                         (uint32_t)seq_bytes, (uint32_t)mask_bytes, (uint32_t)ws_bytes,        \
                         (uint32_t)lo_bytes);                                                  \
  } while (0)
  if (tpr <= 4) SHRIMP_FLN(4);
  else if (tpr <= 8) SHRIMP_FLN(8);
  else if (tpr <= 16) SHRIMP_FLN(16);
  else SHRIMP_FLN(32);
#undef SHRIMP_FLN
  if (int rc = check_launch("trunk_tail/ln")) return rc;
  return launch_value_heads(&k, st);
}

// Pass 2 of the tail: the value / moves-left heads from the head inputs in
// a->workspace (pass 1 or the fused policy tail wrote them).
int shrimp::launch_value_heads(const shrimp_tail_args* a, hipStream_t st) {
  const shrimp_tail_args& k = *a;
  if (!k.value && !k.moves_left) return SHRIMP_OK;
  const int ks1 = kHeadThreads / k.C, ks2 = kHeadThreads / k.bins;
  const size_t smem = ((size_t)kHeadPos * 3 * k.C + (size_t)ks1 * kHeadPos * k.C +
                       (size_t)kHeadPos * k.C + (size_t)ks2 * kHeadPos * k.bins) * sizeof(float);
  hipLaunchKernelGGL(value_head_kernel, dim3((k.B + kHeadPos - 1) / kHeadPos, 2),
                     dim3(kHeadThreads), smem, st, k);
  return check_launch("trunk_tail/heads");
}

// ---- the allocation-free tail ---------------------------------------------------
// The head inputs of shrimp_trunk_tail_noalloc live in this fixed array, one
// copy per device, held until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol):
// the device address comes from hipGetSymbolAddress, once per device with that
// device current, and is kept in scratch_dev.
static __device__ __align__(256) float scratch[SHRIMP_TAIL_SCRATCH_FLOATS];

constexpr int kMaxDevices = 64;
static std::mutex scratch_mu;
static float* scratch_dev[kMaxDevices];

static int scratch_of_current_device(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(SHRIMP_ELAUNCH, "trunk_tail_noalloc: no current device (%d)", dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(SHRIMP_ELAUNCH, "trunk_tail_noalloc: hipGetSymbolAddress: %s",
                       hipGetErrorString(e));
    scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = scratch_dev[dev];
  return SHRIMP_OK;
}

extern "C" int shrimp_trunk_tail(const shrimp_tail_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "trunk_tail: null args");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->workspace, "trunk_tail: null workspace");
  return launch_trunk_tail(a, a->workspace, as_stream(stream));
}

extern "C" int shrimp_trunk_tail_f32(const shrimp_tail_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "trunk_tail_f32: null args");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->workspace, "trunk_tail_f32: null workspace");
  return launch_trunk_tail(a, a->workspace, as_stream(stream), true);
}

extern "C" int shrimp_trunk_tail_noalloc(const shrimp_tail_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "trunk_tail_noalloc: null args");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->B > 0 && a->C > 0, "trunk_tail_noalloc: bad shape (B %d, C %d)", a->B, a->C);
  const int64_t need = mul_sat({a->B, 6, a->C});
  SHRIMP_REQUIRE(need <= (int64_t)SHRIMP_TAIL_SCRATCH_FLOATS,
                 "trunk_tail_noalloc: B * 6 * C = %lld floats exceeds the fixed scratch of %d "
                 "floats (use shrimp_trunk_tail with a workspace)",
                 (long long)need, (int)SHRIMP_TAIL_SCRATCH_FLOATS);
  float* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  return launch_trunk_tail(a, ws, as_stream(stream));
}

extern "C" int shrimp_decode(const float* value_logits, const float* ml_logits,
                             const float* policy, int64_t pol_sb, const int32_t* legal,
                             const int64_t* out_off, int B, int bins, float ml_cap, float* value,
                             float* ml, float* priors, float* logits_out, void* stream) {
  SHRIMP_REQUIRE(B >= 0, "decode: B %d", B);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(value_logits && policy && legal && out_off && value && priors,
                 "decode: null pointer");
  SHRIMP_REQUIRE(!ml_logits || ml, "decode: ml output missing");
  SHRIMP_REQUIRE(bins >= 2 && bins <= 4096, "decode: bins %d", bins);
  SHRIMP_REQUIRE(pol_sb >= 1 && strides_ok({pol_sb}), "decode: policy row stride %lld", (long long)pol_sb);
  hipLaunchKernelGGL(decode_kernel, dim3(B), dim3(256), 0, as_stream(stream), value_logits,
                     ml_logits, policy, pol_sb, legal, out_off, bins, ml_cap, value, ml, priors,
                     logits_out);
  return check_launch("decode");
}

extern "C" int shrimp_build_pair_u8(const int32_t* coords, const uint8_t* mask, const uint8_t* lut,
                                    int lut_m, int B, int N, int n_tokens, int row_ct, int row_tc,
                                    int row_tt, int pad_row, uint8_t* pair, void* stream) {
  SHRIMP_REQUIRE(B >= 0 && N > 0 && N <= 65535 && n_tokens >= 0 && n_tokens <= 4096 && lut_m >= 0 &&
                     lut_m <= 64,
                 "build_pair_u8: bad sizes (B %d, N %d, tokens %d, lut_m %d)", B, N, n_tokens, lut_m);
  SHRIMP_REQUIRE(row_ct >= 0 && row_ct < 256 && row_tc >= 0 && row_tc < 256 && row_tt >= 0 &&
                     row_tt < 256 && pad_row >= 0 && pad_row < 256,
                 "build_pair_u8: rows must fit a byte");
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(coords && mask && lut && pair, "build_pair_u8: null pointer");
  dim3 grid(n_tokens + N, B);
  hipLaunchKernelGGL(pair_kernel, grid, dim3(256), 0, as_stream(stream), coords, mask, lut, lut_m,
                     N, n_tokens, row_ct, row_tc, row_tt, pad_row, pair);
  return check_launch("build_pair_u8");
}

extern "C" int shrimp_build_ray_index(const int32_t* coords, const uint8_t* mask, int B, int N,
                                      int32_t* idx, void* stream) {
  SHRIMP_REQUIRE(B >= 0, "build_ray_index: B %d", B);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(coords && mask && idx, "build_ray_index: null pointer");
  SHRIMP_REQUIRE(N > 0 && N <= RAY_TABLE / 2, "build_ray_index: N %d exceeds %d", N, RAY_TABLE / 2);
  hipLaunchKernelGGL(ray_index_kernel, dim3(B), dim3(256), 0, as_stream(stream), coords, mask, N,
                     idx);
  return check_launch("build_ray_index");
}
