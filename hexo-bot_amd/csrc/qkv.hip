// Fused LayerNorm + q/k/v projection of the attention block for gfx950
// (RelPosAttention.forward, packages/shrimp/python/shrimp/model.py:448-492,
// with AttnBlock's ln1, :508-514):
//
//   n = LN1(seq)  ->  [q | k | v] = n . Wqkv^T + bqkv  ->  (3, B, H, S, dpad) bf16
//
// LN1's affine is folded into the weights at pack time (shrimp_pack_attn_qkv):
//   W' = Wqkv diag(ln_w),  b' = bqkv + Wqkv ln_b,
// so the kernel normalises rows without an affine and feeds them to MFMA in
// bf16. One persistent workgroup per CU keeps the 96 KiB of packed fragments
// (C = 128, 3C outputs) in LDS; each of its 12 waves streams blocks of 16 rows
// (the next block's rows requested before the current block's math), and for
// every 16 outputs (one head's 16 channels when d = 16) writes 16 rows x 32
// bytes of the head-major layout the attention kernel reads.
#include <algorithm>

#include "capi.hpp"
#include "common.hpp"

namespace shrimp {

__global__ void pack_weight_kernel(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                   int K, int NOUT, int cin, int cin_pad, int64_t s_t,
                                   int64_t s_c, int64_t s_n, int interleaved);
__global__ void scale_rows_cols_kernel(const float* __restrict__ src, const float* __restrict__ rs,
                                       const float* __restrict__ cs, int n_out, int n_in,
                                       float* __restrict__ dst);

namespace {

constexpr int QC = QKV_C;                       // channels
constexpr int QN = QKV_N;                       // outputs
constexpr int QWAVES = 12;                      // waves per workgroup (3 per SIMD)
constexpr uint32_t QW_LDS = QKV_W_BYTES;        // 98304 bytes of fragments
constexpr uint32_t QB_OFF = QKV_B_OFF;          // folded bias (fp32) after the fragments
constexpr uint32_t QPACK_BYTES = QKV_PACK_BYTES;

SHRIMP_DEV void load_rows16(const shrimp_qkv_args& a, __amdgpu_buffer_rsrc_t xr, int row, int lg,
                            u32x4 (&xf)[QC / 32]) {
  const uint32_t xo =
      row < a.rows ? (uint32_t)((int64_t)row * a.x_sr * 2) + (uint32_t)(lg * 16) : SHRIMP_OOB_OFFSET;
#pragma unroll
  for (int ks = 0; ks < QC / 32; ++ks) xf[ks] = buf_load16(xr, xo + ks * 64);
}

}  // namespace

// KVF (d = dpad = 16): q keeps the (B, H, S, 16) layout of a.qkv (its first
// plane); k and v go to `kvf` in the staged attention's fragment order, per
// (position, head) SP/16 K fragments then SP/16 V fragments of 512 bytes:
//   K fragment kb, lane (lr, lg): K[16 kb + lr][4 lg .. +3]
//   V fragment kb, lane (lr, lg): V[16 kb + 4 lg .. +3][lr]   (V^T)
// K comes out of the usual product in that order; V from the product with
// the operands swapped (rows as A, weights as B), which leaves each lane four
// consecutive rows of one output channel. Slots of keys >= S are not written.
// Every store goes through a buffer resource, rows that do not exist at an
// offset past it (dropped): with no store under a branch, the wait for the
// next block's rows counts exactly the stores issued after them and never
// waits for those stores.
template <bool KVF>
__global__ __launch_bounds__(QWAVES * 64, 1) void attn_qkv_kernel(const shrimp_qkv_args a,
                                                                  uint32_t x_bytes, int dshift,
                                                                  unsigned short* kvf, int SP,
                                                                  uint32_t q_bytes,
                                                                  uint32_t kvf_bytes) {
  extern __shared__ __attribute__((aligned(16))) unsigned char wl[];
  constexpr int KS = QC / 32, NB = QN / 16;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;

  {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.packed, QW_LDS);
    constexpr int CHUNKS = QW_LDS / 16;
    constexpr int PER = (CHUNKS + QWAVES * 64 - 1) / (QWAVES * 64);
    u32x4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = buf_load16(wr, (uint32_t)(i * QWAVES * 64 + threadIdx.x) * 16);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t off = (uint32_t)(i * QWAVES * 64 + threadIdx.x) * 16;
      if (off < QW_LDS) *reinterpret_cast<u32x4*>(wl + off) = v[i];
    }
  }
  __syncthreads();

  // the folded biases in registers: the block loop issues no bias loads
  BiasRegs<QN / 16> bias;
  const float* pb = reinterpret_cast<const float*>(static_cast<const unsigned char*>(a.packed) + QB_OFF);
  bias.load(pb, lane);
  // the v blocks with columns = channels (KVF: V written transposed): lane
  // (lr, lg) starts all four of its accumulators at bias[16 nb + lr]
  float vcol[QC / 16];
#pragma unroll
  for (int t = 0; t < QC / 16; ++t) vcol[t] = KVF ? pb[16 * (2 * (QC / 16) + t) + lr] : 0.f;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes);
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.qkv, q_bytes);
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(kvf, kvf_bytes);
  const int d = QC / a.H;
  const int64_t plane = (int64_t)a.B * a.H * a.S * a.dpad;  // one of q / k / v
  const int64_t hstride = (int64_t)a.S * a.dpad;

  const int64_t nblk = (a.rows + 15) / 16;
  const int64_t tw = (int64_t)gridDim.x * QWAVES;
  const int64_t gw = (int64_t)blockIdx.x * QWAVES + wave;
  const int begin = (int)(gw * nblk / tw);
  const int end = (int)((gw + 1) * nblk / tw);
  u32x4 cur[KS], nxt[KS];
  if (begin < end) load_rows16(a, xr, begin * 16 + lr, lg, nxt);
  // as many dropped stores (distinct offsets past the resource, so none is
  // merged away) as a block issues after its prefetch: the loop is then
  // entered with the same requests in flight as from its last block, and the
  // wait for the prefetched rows counts the stores instead of waiting for them
#pragma unroll
  for (int i = 0; i < NB; ++i)
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{0u, 0u}, qr, SHRIMP_OOB_OFFSET - i * 256u, 0, 0);
  for (int blk = begin; blk < end; ++blk) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) cur[ks] = nxt[ks];
    load_rows16(a, xr, blk + 1 < end ? (blk + 1) * 16 + lr : a.rows, lg, nxt);
    const int row = blk * 16 + lr;

    // LayerNorm over the 128 channels of this lane's row: 32 in this lane
    // (k = 32 ks + 8 lg + e), the rest in the 3 other lane groups.
    u32x4 hf[KS];
    ln_row128(cur, a.eps, hf);

    // destination of this lane's row in the head-major layout
    const bool rv = row < a.rows;
    const int bq = rv ? row / a.S : 0;
    const int sq = rv ? row - bq * a.S : 0;
    const int64_t rowbase = ((int64_t)bq * a.H * a.S + sq) * a.dpad;  // elements
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      u32x4 w[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        w[ks] = *reinterpret_cast<const u32x4*>(wl + (uint32_t)(((ks * NB + nb) * 64 + lane) * 16));
      const int which = nb / (QC / 16);
      if (KVF && which == 2) {
        // rows 16 blk + 4 lg .. + 3 of output channel 16 (nb - 16) + lr = head nb - 16, dim lr
        const float vb = vcol[nb - 2 * (QC / 16)];
        f32x4 acc = f32x4{vb, vb, vb, vb};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = mfma16x16x32(hf[ks], w[ks], acc);
        const int r0 = blk * 16 + lg * 4;
        const int b0 = r0 < a.rows ? r0 / a.S : 0;
        const int s0 = r0 - b0 * a.S;
        const int head = nb - 2 * (QC / 16);
        const uint32_t off =
            r0 < a.rows ? (uint32_t)(((((int64_t)b0 * a.H + head) * 2 + 1) * SP * 16 + (s0 >> 4) * 256 +
                                      (((s0 & 15) >> 2) * 16 + lr) * 4) * 2)
                        : SHRIMP_OOB_OFFSET;
        __builtin_amdgcn_raw_buffer_store_b64(
            u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])}, kr, off, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      f32x4 acc = bias.rows(nb);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc = mfma16x16x32(w[ks], hf[ks], acc);
      const int within = (nb % (QC / 16)) * 16 + lg * 4;
      const int head = within >> dshift;
      const int dd = within & (d - 1);
      const u32x2 pk{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
      if (KVF && which == 1) {
        const uint32_t off =
            rv ? (uint32_t)(((((int64_t)bq * a.H + head) * 2) * SP * 16 + (sq >> 4) * 256 +
                             (lg * 16 + (sq & 15)) * 4) * 2)
               : SHRIMP_OOB_OFFSET;
        __builtin_amdgcn_raw_buffer_store_b64(pk, kr, off, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      const uint32_t off =
          rv ? (uint32_t)((rowbase + which * plane + head * hstride + dd) * 2) : SHRIMP_OOB_OFFSET;
      __builtin_amdgcn_raw_buffer_store_b64(pk, qr, off, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// b'[n] = b[n] + sum_k W[n][k] ln_b[k]
__global__ void qkv_bias_kernel(const float* __restrict__ w, const float* __restrict__ b,
                                const float* __restrict__ ln_b, float* __restrict__ out) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= QN) return;
  float s = b[n];
  for (int k = 0; k < QC; ++k) s = fmaf(w[(int64_t)n * QC + k], ln_b[k], s);
  out[n] = s;
}

// cs[n] = sum_k W'[n][k] over the packed bf16 fragments (output n = 16 nb + lr
// sits in lane lr + 16 lg of fragment (ks, nb), inputs 32 ks + 8 lg .. +7).
__global__ void qkv_colsum_kernel(const unsigned short* __restrict__ frag, float* __restrict__ cs) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= QN) return;
  const int nb = n / 16, lr = n % 16;
  float s = 0.f;
  for (int ks = 0; ks < QC / 32; ++ks)
    for (int lg = 0; lg < 4; ++lg)
      for (int e = 0; e < 8; ++e)
        s += bf16_bits_to_f32(frag[(((ks * (QN / 16) + nb) * 64) + lg * 16 + lr) * 8 + e]);
  cs[n] = s;
}

}  // namespace shrimp

using namespace shrimp;

extern "C" size_t shrimp_attn_qkv_pack_bytes(int C) { return C == QC ? (size_t)QPACK_BYTES : 0; }

extern "C" int shrimp_pack_attn_qkv(const float* qkv_w, const float* qkv_b, const float* ln_w,
                                    const float* ln_b, void* packed, void* scratch, int C,
                                    void* stream) {
  SHRIMP_REQUIRE(qkv_w && qkv_b && ln_w && ln_b && packed && scratch,
                 "pack_attn_qkv: null pointer");
  SHRIMP_REQUIRE(C == QC, "pack_attn_qkv: fused kernel covers C=%d (got %d)", QC, C);
  hipStream_t st = as_stream(stream);
  float* tmp = static_cast<float*>(scratch);  // 3C * C floats
  unsigned char* pk = static_cast<unsigned char*>(packed);
  const int64_t n = (int64_t)QN * QC;
  hipLaunchKernelGGL(scale_rows_cols_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     qkv_w, (const float*)nullptr, ln_w, QN, QC, tmp);
  const int64_t frags = (int64_t)(QC / 32) * (QN / 16) * 64;
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((frags + 255) / 256)), dim3(256), 0, st,
                     tmp, reinterpret_cast<unsigned short*>(pk), QC, QN, QC, QC, (int64_t)0,
                     (int64_t)1, (int64_t)QC, 0);
  hipLaunchKernelGGL(qkv_bias_kernel, dim3((QN + 255) / 256), dim3(256), 0, st, qkv_w, qkv_b,
                     ln_b, reinterpret_cast<float*>(pk + QB_OFF));
  hipLaunchKernelGGL(qkv_colsum_kernel, dim3((QN + 255) / 256), dim3(256), 0, st,
                     reinterpret_cast<const unsigned short*>(pk), reinterpret_cast<float*>(pk + QKV_CS_OFF));
  return check_launch("pack_attn_qkv");
}

extern "C" int shrimp_attn_qkv(const shrimp_qkv_args* a, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_qkv: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "attn_qkv: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->C == QC, "attn_qkv: fused kernel covers C=%d (got %d)", QC, a->C);
  SHRIMP_REQUIRE(a->x && a->qkv && a->packed, "attn_qkv: null pointer");
  SHRIMP_REQUIRE(a->B > 0 && a->S > 0 && (int64_t)a->B * a->S == a->rows,
                 "attn_qkv: rows must be B * S");
  SHRIMP_REQUIRE(a->H > 0 && QC % a->H == 0, "attn_qkv: C %% H != 0");
  const int d = QC / a->H;
  SHRIMP_REQUIRE(d >= 4 && (d & (d - 1)) == 0 && a->dpad >= d && a->dpad % 4 == 0,
                 "attn_qkv: head dim %d must be a power of two >= 4 with dpad %d >= d", d, a->dpad);
  SHRIMP_REQUIRE(strides_ok({a->x_sr}) && a->x_sr >= QC && a->x_sr % 8 == 0, "attn_qkv: x row stride");
  const int64_t xe = ((int64_t)(a->rows - 1) * a->x_sr + QC) * 2;
  SHRIMP_REQUIRE(xe < (int64_t)0x7FFF0000, "attn_qkv: activation buffer too large");
  const int64_t qe = mul_sat({3, a->B, a->H, a->S, a->dpad, 2});  // q, k and v planes
  SHRIMP_REQUIRE(qe < (int64_t)0x7FFF0000, "attn_qkv: q/k/v buffer too large");
  SHRIMP_REQUIRE((size_t)max_lds_per_block() >= QW_LDS, "attn_qkv: needs %u bytes of LDS",
                 (unsigned)QW_LDS);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return set_error(SHRIMP_ELAUNCH, "attn_qkv: cannot query the compute unit count");
  int dshift = 0;
  while ((1 << dshift) < d) ++dshift;
  const int64_t nblk = (a->rows + 15) / 16;
  // at least one workgroup per 4 row blocks (up to one per compute unit): small
  // row counts spread over more units, each staging the weights once
  const int grid = (int)std::min<int64_t>(cus, std::max<int64_t>((nblk + QWAVES - 1) / QWAVES, (nblk + 3) / 4));
  hipLaunchKernelGGL(attn_qkv_kernel<false>, dim3(grid), dim3(QWAVES * 64), QW_LDS, as_stream(stream),
                     *a, (uint32_t)xe, dshift, (unsigned short*)nullptr, 0, (uint32_t)qe, 0u);
  return check_launch("attn_qkv");
}

extern "C" int shrimp_attn_qkv_kvf(const shrimp_qkv_args* a, void* kvf, void* stream) {
  SHRIMP_REQUIRE(a != nullptr, "attn_qkv_kvf: null args");
  SHRIMP_REQUIRE(a->rows >= 0, "attn_qkv_kvf: negative rows");
  if (a->rows == 0) return SHRIMP_OK;
  SHRIMP_REQUIRE(a->C == QC && a->H == QC / 16 && a->dpad == 16,
                 "attn_qkv_kvf: covers C = %d, H = %d, dpad = 16 (got C = %d, H = %d, dpad = %d)", QC,
                 QC / 16, a->C, a->H, a->dpad);
  SHRIMP_REQUIRE(a->x && a->qkv && a->packed && kvf, "attn_qkv_kvf: null pointer");
  SHRIMP_REQUIRE(a->B > 0 && a->S > 0 && a->S % 4 == 0 && (int64_t)a->B * a->S == a->rows,
                 "attn_qkv_kvf: rows must be B * S with S %% 4 == 0");
  SHRIMP_REQUIRE(strides_ok({a->x_sr}) && a->x_sr >= QC && a->x_sr % 8 == 0, "attn_qkv_kvf: x row stride");
  const int SP = (a->S + 15) & ~15;
  const int64_t xe = ((int64_t)(a->rows - 1) * a->x_sr + QC) * 2;
  const int64_t qe = (int64_t)a->B * a->H * a->S * 16 * 2;  // the q plane
  const int64_t ke = (int64_t)a->B * a->H * SP * 64;       // K and V fragments
  SHRIMP_REQUIRE(xe < (int64_t)0x7FFF0000 && qe < (int64_t)0x7FFF0000 && ke < (int64_t)0x7FFF0000,
                 "attn_qkv_kvf: buffers too large");
  SHRIMP_REQUIRE((size_t)max_lds_per_block() >= QW_LDS, "attn_qkv_kvf: needs %u bytes of LDS",
                 (unsigned)QW_LDS);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return set_error(SHRIMP_ELAUNCH, "attn_qkv_kvf: cannot query the compute unit count");
  const int64_t nblk = (a->rows + 15) / 16;
  const int grid = (int)std::min<int64_t>(cus, std::max<int64_t>((nblk + QWAVES - 1) / QWAVES, (nblk + 3) / 4));
  hipLaunchKernelGGL(attn_qkv_kernel<true>, dim3(grid), dim3(QWAVES * 64), QW_LDS, as_stream(stream),
                     *a, (uint32_t)xe, 4, static_cast<unsigned short*>(kvf), SP, (uint32_t)qe,
                     (uint32_t)ke);
  return check_launch("attn_qkv_kvf");
}
