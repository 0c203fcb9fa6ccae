// AddressSanitizer / UndefinedBehaviorSanitizer driver for the host side of
// the C ABI: the argument checks, the size and offset arithmetic, the launch
// wrappers and the error-text formatting. It links every source file with
// its host side compiled with -fsanitize=address,undefined (the device code is
// compiled unoptimised, only to link: no GPU is visible, so a call that passes
// its checks fails at its launch), and calls
//   - the argument checks the Python tests rely on, with their messages;
//   - every entry point that takes an argument struct with a null struct;
//   - every entry point with many random argument sets drawn from boundary
//     values (sizes around the supported limits, negative and overflowing
//     values, null pointers).
// Each call must return SHRIMP_OK (nothing to do), SHRIMP_EINVAL with a
// message, or SHRIMP_ELAUNCH. Pointer arguments point at a zeroed host
// buffer or are null; host code that read past them would be reported.
//
// Usage: abi_asan [iterations [seed]]. Built by `make -C hexo-bot_amd/csrc
// asan`; tests/test_lib.py runs it on the CPU. It refuses to run where a GPU
// is visible.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>

#include "shrimp_hip.h"

namespace {

int g_failures = 0;
long g_calls = 0, g_ok = 0, g_inval = 0, g_launch = 0;

void expect(bool cond, const char* what) {
  if (!cond) {
    std::fprintf(stderr, "FAIL: %s (last error: %s)\n", what, shrimp_last_error());
    ++g_failures;
  }
}

// Records one call's status: OK, EINVAL (with a message) or ELAUNCH.
void check_rc(int rc, const char* fn) {
  ++g_calls;
  if (rc == SHRIMP_OK) {
    ++g_ok;
  } else if (rc == SHRIMP_EINVAL) {
    ++g_inval;
    if (shrimp_last_error()[0] == '\0') {
      std::fprintf(stderr, "FAIL: %s: EINVAL without a message\n", fn);
      ++g_failures;
    }
  } else if (rc == SHRIMP_ELAUNCH) {
    ++g_launch;
  } else {
    std::fprintf(stderr, "FAIL: %s returned %d\n", fn, rc);
    ++g_failures;
  }
}

void expect_einval(int rc, const char* needle, const char* what) {
  check_rc(rc, what);
  if (rc != SHRIMP_EINVAL || (needle && !std::strstr(shrimp_last_error(), needle))) {
    std::fprintf(stderr, "FAIL: %s: rc %d, message '%s', wanted '%s'\n", what, rc,
                 shrimp_last_error(), needle ? needle : "");
    ++g_failures;
  }
}

// Zeroed host memory behind every non-null pointer argument.
alignas(256) unsigned char g_buf[1 << 16];

struct Fuzz {
  std::mt19937_64 rng;
  explicit Fuzz(uint64_t seed) : rng(seed) {}
  uint64_t u(uint64_t n) { return rng() % n; }
  int32_t i32() {
    static const int32_t pick[] = {-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 12, 15, 16, 17, 24, 31, 32,
                                   33, 48, 64, 80, 96, 127, 128, 129, 136, 192, 255, 256,
                                   257, 264, 320, 321, 368, 384, 464, 512, 513, 576, 577,
                                   1024, 4096, 32767, 65535, 65536, 1 << 20, 0x7FFFFFFF,
                                   -0x7FFFFFFF - 1};
    if (u(8) == 0) return (int32_t)rng();
    return pick[u(sizeof(pick) / sizeof(pick[0]))];
  }
  int64_t i64() {
    static const int64_t pick[] = {0, 1, 7, 8, 16, 32, 64, 128, 256, 264 * 128, 576 * 128,
                                   -1, (int64_t)1 << 31, (int64_t)1 << 40, INT64_MAX};
    if (u(8) == 0) return (int64_t)rng();
    return pick[u(sizeof(pick) / sizeof(pick[0]))];
  }
  float f32() {
    static const float pick[] = {0.f, 1e-5f, 1e-6f, 1.f, -1.f, 64.f,
                                 std::numeric_limits<float>::quiet_NaN(),
                                 std::numeric_limits<float>::infinity()};
    return pick[u(sizeof(pick) / sizeof(pick[0]))];
  }
  void* ptr() { return u(8) == 0 ? nullptr : static_cast<void*>(g_buf); }

  template <class T>
  void set(T*& p) { p = static_cast<T*>(ptr()); }
  void set(int32_t& v) { v = i32(); }
  void set(int64_t& v) { v = i64(); }
  void set(float& v) { v = f32(); }
};

#define FZ(f) fz.set(a.f);

#define CONV_FIELDS(X)                                                                         \
  X(x) X(x_sb) X(x_sn) X(idx) X(taps) X(idx_stride) X(mask) X(w) X(bias) X(ln_w) X(ln_b)      \
  X(eps) X(relu) X(resid) X(r_sb) X(r_sn) X(gamma) X(head_w) X(head_b) X(head_out) X(out)     \
  X(o_sb) X(o_sn) X(B) X(N) X(cin_pad) X(cout)
#define LINEAR_FIELDS(X)                                                                       \
  X(x) X(x_sr) X(w) X(bias) X(ln_w) X(ln_b) X(eps) X(mode) X(resid) X(r_sr) X(gamma) X(mask)  \
  X(out) X(o_sr) X(rows) X(in_features) X(out_features) X(B) X(S) X(H) X(dpad) X(tok_lo)     \
  X(n_tokens)
#define QKV_FIELDS(X) X(x) X(x_sr) X(qkv) X(packed) X(eps) X(rows) X(B) X(S) X(H) X(C) X(dpad)
#define MLPW_FIELDS(X)                                                                         \
  X(out_w) X(out_b) X(g_attn) X(ln_w) X(ln_b) X(fc1_w) X(fc1_b) X(fc2_w) X(fc2_b) X(g_mlp)    \
  X(C) X(hidden)
#define MLP_FIELDS(X)                                                                          \
  X(x) X(x_sr) X(seq) X(s_sr) X(mask) X(packed) X(eps) X(rows) X(C) X(hidden) X(tok_lo) X(S)  \
  X(n_tokens)
#define ATTN_FIELDS(X)                                                                         \
  X(q) X(k) X(v) X(qkv_sb) X(qkv_sh) X(seq_lens) X(pair) X(p_sb) X(p_sq) X(table2)            \
  X(table_rows) X(coords) X(mask) X(btab) X(xtab) X(lut_m) X(n_tokens) X(o) X(o_sb) X(o_sh)   \
  X(o_sr) X(B) X(S) X(H) X(d) X(dpad)
#define PROJ_FIELDS(X) X(x) X(x_sb) X(x_sr) X(packed) X(eps)
#define TAIL_FIELDS(X)                                                                         \
  X(seq) X(s_sb) X(mask) X(ln_w) X(ln_b) X(eps) X(out_seq) X(vr_w) X(vr_b) X(vh_w) X(vh_b)    \
  X(value) X(mr_w) X(mr_b) X(mh_w) X(mh_b) X(moves_left) X(workspace) X(B) X(S) X(n_tokens)  \
  X(C) X(bins) X(tok_lo)
#define RAY_FIELDS(X)                                                                          \
  X(q) X(k) X(v) X(q_sb) X(q_sh) X(q_sn) X(k_sb) X(k_sh) X(k_sn) X(v_sb) X(v_sh) X(v_sn)      \
  X(idx) X(idx_sb) X(idx_sn) X(slot_bias) X(raylen) X(rl_sb) X(rl_sn) X(seq_lens) X(out)      \
  X(o_sb) X(o_sh) X(o_sn) X(B) X(H) X(N) X(D) X(blockers)
#define RAYTAP_FIELDS(X)                                                                       \
  X(x) X(x_sb) X(x_sn) X(gather_idx) X(g_sb) X(g_sn) X(mask) X(packed_w) X(bias) X(ln_w)      \
  X(ln_b) X(ray_idx) X(r_sb) X(r_sn) X(reach) X(re_sb) X(re_sn) X(alpha) X(eps) X(relu)       \
  X(corb) X(out) X(o_sb) X(o_sn) X(B) X(N) X(C) X(Cout)

template <class S>
S zeroed() {
  S s;
  std::memset(&s, 0, sizeof(s));
  return s;
}

// The argument checks tests/test_lib.py also drives through ctypes.
void known_rejections() {
  auto a = zeroed<shrimp_conv_args>();
  a.B = 1; a.N = 4; a.cin_pad = 33; a.cout = 128; a.taps = 7; a.idx_stride = 7; a.x_sn = 64;
  a.x = a.idx = (const int32_t*)g_buf; a.mask = g_buf; a.w = g_buf; a.bias = (const float*)g_buf;
  a.out = g_buf;
  expect_einval(shrimp_hex_conv(&a, nullptr), "cin_pad", "hex_conv cin_pad");
  auto la = zeroed<shrimp_linear_args>();
  la.rows = 4; la.in_features = 100; la.out_features = 128; la.x = la.w = g_buf;
  la.bias = (const float*)g_buf; la.out = g_buf; la.x_sr = 100; la.o_sr = 128;
  expect_einval(shrimp_linear(&la, nullptr), nullptr, "linear in_features");
  auto aa = zeroed<shrimp_attn_args>();
  aa.B = 1; aa.S = 8; aa.H = 2; aa.d = 6; aa.dpad = 16;
  aa.q = aa.k = aa.v = aa.o = g_buf; aa.seq_lens = (const int32_t*)g_buf;
  expect_einval(shrimp_attn(&aa, nullptr), "head dim", "attn head dim");
  expect_einval(shrimp_build_ray_index((const int32_t*)g_buf, g_buf, 1, 5000, (int32_t*)g_buf, nullptr),
                nullptr, "ray index N");
  int64_t one[2] = {0, 0};
  int32_t cnt[4] = {0, 0, 0, 0}, stt[1] = {0};
  expect_einval(shrimp_featurize(nullptr, nullptr, nullptr, one, nullptr, nullptr, 1, 0, 64, nullptr,
                                 nullptr, nullptr, nullptr, cnt, stt, nullptr),
                "radius", "featurize radius");
  auto rt = zeroed<shrimp_raytap_args>();
  rt.B = 1; rt.N = 600; rt.C = 128; rt.Cout = 128; rt.corb = 8;
  expect_einval(shrimp_conv_ln_raytap(&rt, nullptr), "N=600", "raytap N");
  expect(shrimp_raytap_wpack_bytes(96, 96) == (size_t)7 * 96 * 96 * 2, "raytap wpack bytes");
  expect(shrimp_raytap_wpack_bytes(100, 128) == 0, "raytap wpack bytes of an odd C");
  expect(shrimp_attn_fused_supported(128, 8, 321, 16) == 0, "attn_fused S limit");
}

void null_structs() {
  expect_einval(shrimp_hex_conv(nullptr, nullptr), nullptr, "hex_conv null");
  expect_einval(shrimp_hex_conv_f32(nullptr, nullptr), nullptr, "hex_conv_f32 null");
  expect_einval(shrimp_conv_block(nullptr, nullptr, nullptr), nullptr, "conv_block null");
  expect_einval(shrimp_conv_block_pair(nullptr, nullptr, nullptr, nullptr, nullptr), nullptr,
                "conv_block_pair null");
  expect_einval(shrimp_linear(nullptr, nullptr), nullptr, "linear null");
  expect_einval(shrimp_linear_f32(nullptr, nullptr), nullptr, "linear_f32 null");
  expect_einval(shrimp_attn_qkv(nullptr, nullptr), nullptr, "attn_qkv null");
  expect_einval(shrimp_attn_qkv_kvf(nullptr, g_buf, nullptr), nullptr, "attn_qkv_kvf null");
  expect_einval(shrimp_pack_attn_mlp(nullptr, g_buf, g_buf, nullptr), nullptr, "pack_attn_mlp null");
  expect_einval(shrimp_attn_mlp(nullptr, nullptr), nullptr, "attn_mlp null");
  expect_einval(shrimp_attn(nullptr, nullptr), nullptr, "attn null");
  expect_einval(shrimp_attn_f32(nullptr, nullptr), nullptr, "attn_f32 null");
  expect_einval(shrimp_attn_fused(nullptr, nullptr, nullptr), nullptr, "attn_fused null");
  expect_einval(shrimp_attn_staged(nullptr, g_buf, (const int32_t*)g_buf, nullptr), nullptr,
                "attn_staged null");
  expect_einval(shrimp_trunk_tail(nullptr, nullptr), nullptr, "trunk_tail null");
  expect_einval(shrimp_trunk_tail_f32(nullptr, nullptr), nullptr, "trunk_tail_f32 null");
  expect_einval(shrimp_trunk_tail_noalloc(nullptr, nullptr), nullptr, "trunk_tail_noalloc null");
  expect_einval(shrimp_policy_tail(nullptr, nullptr, nullptr), nullptr, "policy_tail null");
  expect_einval(shrimp_ray_attn(nullptr, nullptr), nullptr, "ray_attn null");
  expect_einval(shrimp_conv_ln_raytap(nullptr, nullptr), nullptr, "conv_ln_raytap null");
}

void fuzz_structs(uint64_t seed, int iters) {
  Fuzz fz(seed);
  for (int it = 0; it < iters; ++it) {
    {
      shrimp_conv_args a; CONV_FIELDS(FZ)
      check_rc(shrimp_hex_conv(&a, nullptr), "hex_conv");
      check_rc(shrimp_hex_conv_f32(&a, nullptr), "hex_conv_f32");
      shrimp_conv_args c2 = a; c2.resid = a.x; c2.gamma = a.bias;
      check_rc(shrimp_conv_block(&a, &c2, nullptr), "conv_block");
      check_rc(shrimp_conv_block_pair(&a, &c2, &a, &c2, nullptr), "conv_block_pair");
      shrimp_tail_args t; { auto& a = t; TAIL_FIELDS(FZ) }
      check_rc(shrimp_policy_tail(&a, &t, nullptr), "policy_tail");
    }
    {
      shrimp_linear_args a; LINEAR_FIELDS(FZ)
      check_rc(shrimp_linear(&a, nullptr), "linear");
      check_rc(shrimp_linear_f32(&a, nullptr), "linear_f32");
    }
    {
      shrimp_qkv_args a; QKV_FIELDS(FZ)
      check_rc(shrimp_attn_qkv(&a, nullptr), "attn_qkv");
      check_rc(shrimp_attn_qkv_kvf(&a, fz.ptr(), nullptr), "attn_qkv_kvf");
    }
    {
      shrimp_mlp_weights a; MLPW_FIELDS(FZ)
      check_rc(shrimp_pack_attn_mlp(&a, fz.ptr(), fz.ptr(), nullptr), "pack_attn_mlp");
    }
    {
      shrimp_mlp_args a; MLP_FIELDS(FZ)
      check_rc(shrimp_attn_mlp(&a, nullptr), "attn_mlp");
    }
    {
      shrimp_attn_args a; ATTN_FIELDS(FZ)
      check_rc(shrimp_attn(&a, nullptr), "attn");
      check_rc(shrimp_attn_f32(&a, nullptr), "attn_f32");
      check_rc(shrimp_attn_staged(&a, fz.ptr(), (const int32_t*)fz.ptr(), nullptr), "attn_staged");
      shrimp_attn_proj_args p; { auto& a = p; PROJ_FIELDS(FZ) }
      check_rc(shrimp_attn_fused(&a, &p, nullptr), "attn_fused");
    }
    {
      shrimp_tail_args a; TAIL_FIELDS(FZ)
      check_rc(shrimp_trunk_tail(&a, nullptr), "trunk_tail");
      check_rc(shrimp_trunk_tail_f32(&a, nullptr), "trunk_tail_f32");
      check_rc(shrimp_trunk_tail_noalloc(&a, nullptr), "trunk_tail_noalloc");
    }
    {
      shrimp_ray_attn_args a; RAY_FIELDS(FZ)
      check_rc(shrimp_ray_attn(&a, nullptr), "ray_attn");
    }
    {
      shrimp_raytap_args a; RAYTAP_FIELDS(FZ)
      check_rc(shrimp_conv_ln_raytap(&a, nullptr), "conv_ln_raytap");
    }
  }
}

void fuzz_scalars(uint64_t seed, int iters) {
  Fuzz fz(seed);
  auto P = [&]() { return fz.ptr(); };
  for (int it = 0; it < iters; ++it) {
    const int i0 = fz.i32(), i1 = fz.i32(), i2 = fz.i32(), i3 = fz.i32(), i4 = fz.i32();
    (void)shrimp_conv_wpack_bytes(i0, i1, i2);
    (void)shrimp_conv_wpack_bytes_f32(i0, i1, i2);
    (void)shrimp_linear_wpack_bytes(i0, i1);
    (void)shrimp_attn_qkv_pack_bytes(i0);
    (void)shrimp_attn_mlp_pack_bytes(i0, i1);
    (void)shrimp_attn_keys_bytes(i0);
    (void)shrimp_raytap_wpack_bytes(i0, i1);
    (void)shrimp_conv_block_supported(i0, i1, i2, i3);
    (void)shrimp_conv_block_pair_supported(i0, i1, i2, i3);
    (void)shrimp_policy_tail_supported(i0, i1);
    (void)shrimp_attn_fused_supported(i0, i1, i2, i3);
    (void)shrimp_attn_staged_supported(i0, i1, i2);
    check_rc(shrimp_pack_conv_weight((const float*)P(), P(), i0, i1, i2, i3, nullptr), "pack_conv_weight");
    check_rc(shrimp_pack_conv_weight_f32((const float*)P(), (float*)P(), i0, i1, i2, i3, nullptr),
             "pack_conv_weight_f32");
    check_rc(shrimp_pack_linear_weight((const float*)P(), P(), i0, i1, nullptr), "pack_linear_weight");
    check_rc(shrimp_pack_linear_weight_f32((const float*)P(), (float*)P(), i0, i1, nullptr),
             "pack_linear_weight_f32");
    check_rc(shrimp_pack_attn_qkv((const float*)P(), (const float*)P(), (const float*)P(),
                                  (const float*)P(), P(), P(), i0, nullptr),
             "pack_attn_qkv");
    check_rc(shrimp_attn_keys((const int32_t*)P(), (const uint8_t*)P(), (const int32_t*)P(), i0, i1, i2,
                              (int32_t*)P(), nullptr),
             "attn_keys");
    check_rc(shrimp_attn_bias_table((const float*)P(), i0, i1, (const uint8_t*)P(), i2, i3, i4, fz.i32(),
                                    (float*)P(), P(), nullptr),
             "attn_bias_table");
    check_rc(shrimp_prep_inputs(P(), (int)fz.u(7), P(), P(), (int)fz.u(7), P(), (int)fz.u(7), i0, i1, i2,
                                i3, (int32_t*)P(), (uint8_t*)P(), (int32_t*)P(), (int32_t*)P(),
                                (uint8_t*)P(), P(), nullptr),
             "prep_inputs");
    check_rc(shrimp_prep_csr(P(), i0, (const int16_t*)P(), (const uint16_t*)P(), (const int64_t*)P(), i1,
                             i2, i3, i4, (int32_t*)P(), (uint8_t*)P(), (int32_t*)P(), (int32_t*)P(),
                             (uint8_t*)P(), P(), nullptr),
             "prep_csr");
    check_rc(shrimp_fill_tokens((const float*)P(), i0, i1, P(), fz.i64(), P(), i2, nullptr), "fill_tokens");
    check_rc(shrimp_fill_tokens_f32((const float*)P(), i0, i1, (float*)P(), fz.i64(), i2, nullptr),
             "fill_tokens_f32");
    check_rc(shrimp_featurize((const int32_t*)P(), (const uint8_t*)P(), (const int32_t*)P(),
                              (const int64_t*)P(), (const uint8_t*)P(), (const uint8_t*)P(), i0, i1, i2,
                              (float*)P(), (int32_t*)P(), (uint8_t*)P(), (int32_t*)P(), (int32_t*)P(),
                              (int32_t*)P(), nullptr),
             "featurize");
    check_rc(shrimp_decode((const float*)P(), (const float*)P(), (const float*)P(), fz.i64(),
                           (const int32_t*)P(), (const int64_t*)P(), i0, i1, fz.f32(), (float*)P(),
                           (float*)P(), (float*)P(), (float*)P(), nullptr),
             "decode");
    check_rc(shrimp_build_pair_u8((const int32_t*)P(), (const uint8_t*)P(), (const uint8_t*)P(), i0, i1,
                                  i2, i3, i4, fz.i32(), fz.i32(), fz.i32(), (uint8_t*)P(), nullptr),
             "build_pair_u8");
    check_rc(shrimp_build_ray_index((const int32_t*)P(), (const uint8_t*)P(), i0, i1, (int32_t*)P(), nullptr),
             "build_ray_index");
    check_rc(shrimp_pack_raytap_weight((const uint16_t*)P(), i0, i1, P(), nullptr), "pack_raytap_weight");
    check_rc(shrimp_prep_feats_f32(P(), (int)fz.u(7), i0, i1, i2, (float*)P(), nullptr), "prep_feats_f32");
    check_rc(shrimp_prep_csr_feats_f32(P(), i0, (const int64_t*)P(), i1, i2, i3, (float*)P(), nullptr),
             "prep_csr_feats_f32");
    // the release host side has no phase stamps: every unit is refused
    expect_einval(shrimp_phase_clock(P(), (int)fz.u(4) - 1), "phase", "phase_clock");
    // process-wide switches: out-of-range values only query
    const int cv = shrimp_conv_variant(-1), av = shrimp_attn_variant(-1), rv = shrimp_ray_attn_variant(-1);
    expect(shrimp_conv_variant(i0 > 3 || i0 < 0 ? i0 : 99) == cv, "conv_variant query");
    expect(shrimp_attn_variant(i1 > 3 || i1 < 0 ? i1 : 99) == av, "attn_variant query");
    expect(shrimp_ray_attn_variant(i2 > 3 || i2 < 0 ? i2 : 99) == rv, "ray_attn_variant query");
  }
}

}  // namespace

int main(int argc, char** argv) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) == hipSuccess && ndev > 0) {
    std::fprintf(stderr, "abi_asan: %d GPU(s) visible; this driver hands host buffers to the launch "
                         "wrappers and runs only where no GPU is visible\n", ndev);
    return 2;
  }
  const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
  const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 20261202;
  expect(shrimp_abi_version() == SHRIMP_ABI_VERSION, "abi version");
  known_rejections();
  null_structs();
  fuzz_structs(seed, iters);
  fuzz_scalars(seed + 1, iters);
  std::printf("abi_asan: %ld calls: %ld ok, %ld rejected, %ld reached a launch; %d failures\n", g_calls,
              g_ok, g_inval, g_launch, g_failures);
  return g_failures == 0 ? 0 : 1;
}
