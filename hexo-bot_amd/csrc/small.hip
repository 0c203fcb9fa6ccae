// Small per-position kernels around the Shrimp forward: input preparation,
// token rows, the trunk tail (final LayerNorm + pooled value head), serve
// decode, and the pair / ray index builders. One workgroup per position; all
// are bandwidth-trivial next to the conv and attention kernels.
#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

__device__ __forceinline__ int64_t load_index(const void* p, int dt, int64_t i) {
  switch (dt) {
    case SHRIMP_DT_I64: return static_cast<const int64_t*>(p)[i];
    case SHRIMP_DT_I32: return static_cast<const int32_t*>(p)[i];
    case SHRIMP_DT_U16: {
      const unsigned v = static_cast<const uint16_t*>(p)[i];
      return v == 0xFFFFu ? -1 : (int64_t)v;
    }
    default: return -1;
  }
}

__device__ __forceinline__ float load_feat(const void* p, int dt, int64_t i) {
  switch (dt) {
    case SHRIMP_DT_F32: return static_cast<const float*>(p)[i];
    case SHRIMP_DT_F16: return (float)static_cast<const _Float16*>(p)[i];
    case SHRIMP_DT_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    default: return 0.f;
  }
}

// ---- input preparation (model.py:861-863, 884-892; batching.py:264-276) --------
__global__ __launch_bounds__(256) void prep_kernel(const void* nbr, int nbr_dt, const void* mask,
                                                   const void* coords, int coords_dt,
                                                   const void* feats, int feats_dt, int nfeat,
                                                   int N, int n_tokens, int32_t* idx,
                                                   uint8_t* mask8, int32_t* coords32,
                                                   int32_t* seq_lens, uint8_t* seq_mask,
                                                   uint16_t* xin) {
  const int b = blockIdx.x;
  const int64_t base = (int64_t)b * N;
  if (seq_mask)
    for (int t = threadIdx.x; t < n_tokens; t += blockDim.x)
      seq_mask[(int64_t)b * (n_tokens + N) + t] = 1;
  int last = 0;  // 1 + index of the last live cell
  for (int n = threadIdx.x; n < N; n += blockDim.x) {
    const int64_t r = base + n;
    const bool live = static_cast<const uint8_t*>(mask)[r] != 0;
    if (live) last = n + 1;
    if (mask8) mask8[r] = live ? 1 : 0;
    if (seq_mask) seq_mask[(int64_t)b * (n_tokens + N) + n_tokens + n] = live ? 1 : 0;
    if (idx) {
      idx[r * 7] = n;
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const int64_t j = load_index(nbr, nbr_dt, r * 6 + k);
        idx[r * 7 + 1 + k] = (j >= 0 && j < N) ? (int32_t)j : N;
      }
    }
    if (coords32) {
      coords32[r * 2] = (int32_t)load_index(coords, coords_dt, r * 2);
      coords32[r * 2 + 1] = (int32_t)load_index(coords, coords_dt, r * 2 + 1);
    }
    if (xin) {
#pragma unroll 4
      for (int f = 0; f < 32; f += 2) {
        const float v0 = f < nfeat ? load_feat(feats, feats_dt, r * nfeat + f) : 0.f;
        const float v1 = f + 1 < nfeat ? load_feat(feats, feats_dt, r * nfeat + f + 1) : 0.f;
        reinterpret_cast<unsigned*>(xin + r * 32)[f / 2] = pack_bf16x2(v0, v1);
      }
    }
  }
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

__global__ void fill_tokens_kernel(const float* __restrict__ tokens, int n_tokens, int C,
                                   uint16_t* __restrict__ seq, int64_t seq_sb) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < n_tokens * C; i += blockDim.x)
    seq[(int64_t)b * seq_sb + i] = f32_to_bf16_bits(tokens[i]);
}

// ---- trunk tail + value heads (model.py:927-935, 990-1002) --------------------
// Pass 1, one workgroup per position: final LayerNorm of every row (cells
// masked), written to out_seq; the value-head inputs [T0 | T1 | pooled] and
// [T4 | T5 | pooled] go to the workspace (B, 6C) fp32. Each wave keeps four
// rows in flight; a lane owns channel pairs (2 lane + 128 u, +1).
__global__ __launch_bounds__(256) void final_ln_kernel(const shrimp_tail_args a) {
  __shared__ float pool_w[4][256];
  __shared__ int cnt_w[4];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int C = a.C, S = a.S, nt = a.n_tokens, N = S - nt;
  const uint16_t* seq = static_cast<const uint16_t*>(a.seq) + (int64_t)b * a.s_sb;
  uint16_t* outs = static_cast<uint16_t*>(a.out_seq) + (int64_t)b * a.s_sb;
  float* vin = a.workspace + (int64_t)b * 6 * C;
  float lw[2][2], lb[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = 2 * lane + 128 * u + e;
      lw[u][e] = c < C ? a.ln_w[c] : 0.f;
      lb[u][e] = c < C ? a.ln_b[c] : 0.f;
    }
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  int cnt = 0;
  for (int row0 = wave * 4; row0 < S; row0 += 16) {
    unsigned raw[4][2];
    bool live[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + r;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = 2 * lane + 128 * u;
        raw[r][u] = (row < S && c < C)
                        ? *reinterpret_cast<const unsigned*>(seq + (int64_t)row * C + c)
                        : 0u;
      }
      live[r] = row < S && (row < nt || a.mask[(int64_t)b * N + (row - nt)] != 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + r;
      if (row >= S) break;  // wave-uniform
      float x[2][2];
      float sum = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        x[u][0] = bf16_lo(raw[r][u]);
        x[u][1] = bf16_hi(raw[r][u]);
        sum += x[u][0] + x[u][1];
      }
      const float mean = wave_sum(sum) / C;
      float q = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int c = 2 * lane + 128 * u + e;
          x[u][e] = c < C ? x[u][e] - mean : 0.f;
          q += x[u][e] * x[u][e];
        }
      const float rstd = rsqrtf(wave_sum(q) / C + a.eps);
      const bool is_cell = row >= nt;
      if (is_cell && live[r]) ++cnt;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = 2 * lane + 128 * u;
        if (c >= C) continue;
        float y0 = x[u][0] * rstd * lw[u][0] + lb[u][0];
        float y1 = x[u][1] * rstd * lw[u][1] + lb[u][1];
        if (!live[r]) y0 = y1 = 0.f;
        *reinterpret_cast<unsigned*>(outs + (int64_t)row * C + c) = pack_bf16x2(y0, y1);
        if (is_cell) {
          acc[u][0] += y0;
          acc[u][1] += y1;
        }
        // token rows 0, 1 feed the value head, rows 4, 5 the moves-left head
        const int slot = row == 0 ? 0 : row == 1 ? 1 : row == 4 ? 3 : row == 5 ? 4 : -1;
        if (slot >= 0) {
          vin[slot * C + c] = y0;
          vin[slot * C + c + 1] = y1;
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = 2 * lane + 128 * u + e;
      if (c < C) pool_w[wave][c] = acc[u][e];
    }
  if (lane == 0) cnt_w[wave] = cnt;
  __syncthreads();
  const float inv = 1.0f / (float)max(1, cnt_w[0] + cnt_w[1] + cnt_w[2] + cnt_w[3]);
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const float p = (pool_w[0][c] + pool_w[1][c] + pool_w[2][c] + pool_w[3][c]) * inv;
    vin[2 * C + c] = p;
    vin[5 * C + c] = p;
  }
}

// Pass 2: value / moves-left heads for 4 positions per workgroup; weights are
// transposed (k-major) so a wave's weight load covers 64 consecutive outputs.
constexpr int kHeadPos = 4;
__global__ __launch_bounds__(256) void value_head_kernel(const shrimp_tail_args a) {
  extern __shared__ float hs[];
  const int C = a.C, bins = a.bins;
  float* in = hs;                   // [kHeadPos][3C]
  float* hid = hs + kHeadPos * 3 * C;  // [kHeadPos][C]
  const int b0 = blockIdx.x * kHeadPos;
  const int np = min(kHeadPos, a.B - b0);
  for (int pass = 0; pass < 2; ++pass) {
    const float* rwt = pass == 0 ? a.vr_w : a.mr_w;
    const float* rb = pass == 0 ? a.vr_b : a.mr_b;
    const float* hwt = pass == 0 ? a.vh_w : a.mh_w;
    const float* hb = pass == 0 ? a.vh_b : a.mh_b;
    float* dst = pass == 0 ? a.value : a.moves_left;
    if (dst == nullptr) continue;  // uniform
    for (int i = threadIdx.x; i < kHeadPos * 3 * C; i += blockDim.x) {
      const int p = i / (3 * C), k = i - p * 3 * C;
      in[i] = p < np ? a.workspace[(int64_t)(b0 + p) * 6 * C + pass * 3 * C + k] : 0.f;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < C; o += blockDim.x) {
      float s[kHeadPos] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = 0; k < 3 * C; ++k) {
        const float w = rwt[(int64_t)k * C + o];
#pragma unroll
        for (int p = 0; p < kHeadPos; ++p) s[p] += w * in[p * 3 * C + k];
      }
#pragma unroll
      for (int p = 0; p < kHeadPos; ++p) hid[p * C + o] = fmaxf(s[p] + rb[o], 0.f);
    }
    __syncthreads();
    for (int o = threadIdx.x; o < bins; o += blockDim.x) {
      float s[kHeadPos] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = 0; k < C; ++k) {
        const float w = hwt[(int64_t)k * bins + o];
#pragma unroll
        for (int p = 0; p < kHeadPos; ++p) s[p] += w * hid[p * C + k];
      }
#pragma unroll
      for (int p = 0; p < kHeadPos; ++p)
        if (p < np) dst[(int64_t)(b0 + p) * bins + o] = s[p] + hb[o];
    }
    __syncthreads();
  }
}

// ---- serve decode (inference.py:998-1042, losses.py:40-60) ---------------------
__device__ float block_reduce(float v, bool is_max, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  SHRIMP_REQUIRE(B >= 0 && N > 0, "prep_inputs: bad shape (%d, %d)", B, N);
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(mask != nullptr, "prep_inputs: mask required");
  SHRIMP_REQUIRE(!idx || (nbr && (nbr_dt == SHRIMP_DT_I64 || nbr_dt == SHRIMP_DT_I32 ||
                                  nbr_dt == SHRIMP_DT_U16)),
                 "prep_inputs: nbr dtype");
  SHRIMP_REQUIRE(!coords32 || (coords && (coords_dt == SHRIMP_DT_I64 || coords_dt == SHRIMP_DT_I32)),
                 "prep_inputs: coords dtype");
  SHRIMP_REQUIRE(!xin || (feats && nfeat > 0 && nfeat <= 32 &&
                          (feats_dt == SHRIMP_DT_F32 || feats_dt == SHRIMP_DT_F16 ||
                           feats_dt == SHRIMP_DT_BF16)),
                 "prep_inputs: feats dtype / width");
  hipLaunchKernelGGL(prep_kernel, dim3(B), dim3(256), 0, as_stream(stream), nbr, nbr_dt, mask,
                     coords, coords_dt, feats, feats_dt, nfeat, N, n_tokens, idx, mask8, coords32,
                     seq_lens, seq_mask, static_cast<uint16_t*>(xin));
  return check_launch("prep_inputs");
}

extern "C" int shrimp_fill_tokens(const float* tokens, int n_tokens, int C, void* seq,
                                  int64_t seq_sb, int B, void* stream) {
  SHRIMP_REQUIRE(tokens && seq, "fill_tokens: null pointer");
  if (B == 0 || n_tokens == 0) return SHRIMP_OK;
  hipLaunchKernelGGL(fill_tokens_kernel, dim3(B), dim3(256), 0, as_stream(stream), tokens,
                     n_tokens, C, static_cast<uint16_t*>(seq), seq_sb);
  return check_launch("fill_tokens");
}

extern "C" int shrimp_trunk_tail(const shrimp_tail_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "trunk_tail: null args");
  if (a->B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->seq && a->mask && a->ln_w && a->ln_b && a->out_seq && a->workspace,
                 "trunk_tail: null pointer");
  SHRIMP_REQUIRE(a->C > 0 && a->C <= 256 && a->C % 2 == 0, "trunk_tail: C %d outside (0, 256]",
                 a->C);
  SHRIMP_REQUIRE(a->s_sb % 2 == 0, "trunk_tail: position stride must be even");
  SHRIMP_REQUIRE(a->n_tokens >= 6 && a->S > a->n_tokens, "trunk_tail: needs >= 6 tokens");
  SHRIMP_REQUIRE(!a->value || (a->vr_w && a->vr_b && a->vh_w && a->vh_b), "trunk_tail: value head");
  SHRIMP_REQUIRE(!a->moves_left || (a->mr_w && a->mr_b && a->mh_w && a->mh_b),
                 "trunk_tail: moves-left head");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(final_ln_kernel, dim3(a->B), dim3(256), 0, st, *a);
  if (int rc = check_launch("trunk_tail/ln")) return rc;
  if (!a->value && !a->moves_left) return SHRIMP_OK;
  const size_t smem = (size_t)kHeadPos * 4 * a->C * sizeof(float);
  hipLaunchKernelGGL(value_head_kernel, dim3((a->B + kHeadPos - 1) / kHeadPos), dim3(256), smem,
                     st, *a);
  return check_launch("trunk_tail/heads");
}

extern "C" int shrimp_decode(const float* value_logits, const float* ml_logits,
                             const float* policy, int64_t pol_sb, const int32_t* legal,
                             const int64_t* out_off, int B, int bins, float ml_cap, float* value,
                             float* ml, float* priors, float* logits_out, void* stream) {
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(value_logits && policy && legal && out_off && value && priors,
                 "decode: null pointer");
  SHRIMP_REQUIRE(!ml_logits || ml, "decode: ml output missing");
  SHRIMP_REQUIRE(bins >= 2, "decode: bins %d", bins);
  hipLaunchKernelGGL(decode_kernel, dim3(B), dim3(256), 0, as_stream(stream), value_logits,
                     ml_logits, policy, pol_sb, legal, out_off, bins, ml_cap, value, ml, priors,
                     logits_out);
  return check_launch("decode");
}

extern "C" int shrimp_build_pair_u8(const int32_t* coords, const uint8_t* mask, const uint8_t* lut,
                                    int lut_m, int B, int N, int n_tokens, int row_ct, int row_tc,
                                    int row_tt, int pad_row, uint8_t* pair, void* stream) {
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(coords && mask && lut && pair, "build_pair_u8: null pointer");
  dim3 grid(n_tokens + N, B);
  hipLaunchKernelGGL(pair_kernel, grid, dim3(256), 0, as_stream(stream), coords, mask, lut, lut_m,
                     N, n_tokens, row_ct, row_tc, row_tt, pad_row, pair);
  return check_launch("build_pair_u8");
}

extern "C" int shrimp_build_ray_index(const int32_t* coords, const uint8_t* mask, int B, int N,
                                      int32_t* idx, void* stream) {
  if (B == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(coords && mask && idx, "build_ray_index: null pointer");
  SHRIMP_REQUIRE(N > 0 && 2 * N <= RAY_TABLE, "build_ray_index: N %d exceeds %d", N, RAY_TABLE / 2);
  hipLaunchKernelGGL(ray_index_kernel, dim3(B), dim3(256), 0, as_stream(stream), coords, mask, N,
                     idx);
  return check_launch("build_ray_index");
}
