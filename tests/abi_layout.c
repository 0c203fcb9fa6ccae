/* Prints sizeof / offsetof of every C-ABI struct so tests/test_lib.py can
 * compare them with the ctypes mirrors in shrimp/_lib.py. */
#include <stddef.h>
#include <stdio.h>

#include "shrimp_hip.h"

#define F(S, f) printf("%s.%s %zu\n", #S, #f, offsetof(S, f))
#define Z(S) printf("%s.__size__ %zu\n", #S, sizeof(S))

int main(void) {
  Z(shrimp_conv_args);
  F(shrimp_conv_args, x); F(shrimp_conv_args, x_sb); F(shrimp_conv_args, x_sn);
  F(shrimp_conv_args, idx); F(shrimp_conv_args, taps); F(shrimp_conv_args, idx_stride);
  F(shrimp_conv_args, mask); F(shrimp_conv_args, w); F(shrimp_conv_args, bias);
  F(shrimp_conv_args, ln_w); F(shrimp_conv_args, ln_b); F(shrimp_conv_args, eps);
  F(shrimp_conv_args, relu); F(shrimp_conv_args, resid); F(shrimp_conv_args, r_sb);
  F(shrimp_conv_args, r_sn); F(shrimp_conv_args, gamma); F(shrimp_conv_args, head_w);
  F(shrimp_conv_args, head_b); F(shrimp_conv_args, head_out); F(shrimp_conv_args, out);
  F(shrimp_conv_args, o_sb); F(shrimp_conv_args, o_sn); F(shrimp_conv_args, B);
  F(shrimp_conv_args, N); F(shrimp_conv_args, cin_pad); F(shrimp_conv_args, cout);
  Z(shrimp_linear_args);
  F(shrimp_linear_args, x); F(shrimp_linear_args, x_sr); F(shrimp_linear_args, w);
  F(shrimp_linear_args, bias); F(shrimp_linear_args, ln_w); F(shrimp_linear_args, ln_b);
  F(shrimp_linear_args, eps); F(shrimp_linear_args, mode); F(shrimp_linear_args, resid);
  F(shrimp_linear_args, r_sr); F(shrimp_linear_args, gamma); F(shrimp_linear_args, mask);
  F(shrimp_linear_args, out); F(shrimp_linear_args, o_sr); F(shrimp_linear_args, rows);
  F(shrimp_linear_args, in_features); F(shrimp_linear_args, out_features);
  F(shrimp_linear_args, B); F(shrimp_linear_args, S); F(shrimp_linear_args, H);
  F(shrimp_linear_args, dpad); F(shrimp_linear_args, tok_lo); F(shrimp_linear_args, n_tokens);
  Z(shrimp_attn_args);
  F(shrimp_attn_args, q); F(shrimp_attn_args, k); F(shrimp_attn_args, v);
  F(shrimp_attn_args, qkv_sb); F(shrimp_attn_args, qkv_sh); F(shrimp_attn_args, seq_lens);
  F(shrimp_attn_args, pair); F(shrimp_attn_args, p_sb); F(shrimp_attn_args, p_sq);
  F(shrimp_attn_args, table2); F(shrimp_attn_args, table_rows); F(shrimp_attn_args, coords);
  F(shrimp_attn_args, mask); F(shrimp_attn_args, btab); F(shrimp_attn_args, xtab); F(shrimp_attn_args, lut_m);
  F(shrimp_attn_args, n_tokens); F(shrimp_attn_args, o); F(shrimp_attn_args, o_sb);
  F(shrimp_attn_args, o_sh); F(shrimp_attn_args, o_sr); F(shrimp_attn_args, B);
  F(shrimp_attn_args, S); F(shrimp_attn_args, H); F(shrimp_attn_args, d);
  F(shrimp_attn_args, dpad);
  Z(shrimp_attn_proj_args);
  F(shrimp_attn_proj_args, x); F(shrimp_attn_proj_args, x_sb); F(shrimp_attn_proj_args, x_sr);
  F(shrimp_attn_proj_args, packed); F(shrimp_attn_proj_args, eps);
  Z(shrimp_tail_args);
  F(shrimp_tail_args, seq); F(shrimp_tail_args, s_sb); F(shrimp_tail_args, mask);
  F(shrimp_tail_args, ln_w); F(shrimp_tail_args, ln_b); F(shrimp_tail_args, eps);
  F(shrimp_tail_args, out_seq); F(shrimp_tail_args, vr_w); F(shrimp_tail_args, vr_b);
  F(shrimp_tail_args, vh_w); F(shrimp_tail_args, vh_b); F(shrimp_tail_args, value);
  F(shrimp_tail_args, mr_w); F(shrimp_tail_args, mr_b); F(shrimp_tail_args, mh_w);
  F(shrimp_tail_args, mh_b); F(shrimp_tail_args, moves_left); F(shrimp_tail_args, workspace);
  F(shrimp_tail_args, B);
  F(shrimp_tail_args, S); F(shrimp_tail_args, n_tokens); F(shrimp_tail_args, C);
  F(shrimp_tail_args, bins); F(shrimp_tail_args, tok_lo);
  Z(shrimp_qkv_args);
  F(shrimp_qkv_args, x); F(shrimp_qkv_args, x_sr); F(shrimp_qkv_args, qkv);
  F(shrimp_qkv_args, packed); F(shrimp_qkv_args, eps); F(shrimp_qkv_args, rows);
  F(shrimp_qkv_args, B); F(shrimp_qkv_args, S); F(shrimp_qkv_args, H); F(shrimp_qkv_args, C);
  F(shrimp_qkv_args, dpad);
  Z(shrimp_mlp_weights);
  F(shrimp_mlp_weights, out_w); F(shrimp_mlp_weights, out_b); F(shrimp_mlp_weights, g_attn);
  F(shrimp_mlp_weights, ln_w); F(shrimp_mlp_weights, ln_b); F(shrimp_mlp_weights, fc1_w);
  F(shrimp_mlp_weights, fc1_b); F(shrimp_mlp_weights, fc2_w); F(shrimp_mlp_weights, fc2_b);
  F(shrimp_mlp_weights, g_mlp); F(shrimp_mlp_weights, C); F(shrimp_mlp_weights, hidden);
  Z(shrimp_mlp_args);
  F(shrimp_mlp_args, x); F(shrimp_mlp_args, x_sr); F(shrimp_mlp_args, seq);
  F(shrimp_mlp_args, s_sr); F(shrimp_mlp_args, mask); F(shrimp_mlp_args, packed);
  F(shrimp_mlp_args, eps); F(shrimp_mlp_args, rows); F(shrimp_mlp_args, C);
  F(shrimp_mlp_args, hidden); F(shrimp_mlp_args, tok_lo); F(shrimp_mlp_args, S);
  F(shrimp_mlp_args, n_tokens);
  Z(shrimp_ray_attn_args);
  F(shrimp_ray_attn_args, q); F(shrimp_ray_attn_args, k); F(shrimp_ray_attn_args, v);
  F(shrimp_ray_attn_args, q_sb); F(shrimp_ray_attn_args, q_sh); F(shrimp_ray_attn_args, q_sn);
  F(shrimp_ray_attn_args, k_sb); F(shrimp_ray_attn_args, k_sh); F(shrimp_ray_attn_args, k_sn);
  F(shrimp_ray_attn_args, v_sb); F(shrimp_ray_attn_args, v_sh); F(shrimp_ray_attn_args, v_sn);
  F(shrimp_ray_attn_args, idx); F(shrimp_ray_attn_args, idx_sb); F(shrimp_ray_attn_args, idx_sn);
  F(shrimp_ray_attn_args, slot_bias); F(shrimp_ray_attn_args, raylen);
  F(shrimp_ray_attn_args, rl_sb); F(shrimp_ray_attn_args, rl_sn); F(shrimp_ray_attn_args, seq_lens);
  F(shrimp_ray_attn_args, out); F(shrimp_ray_attn_args, o_sb); F(shrimp_ray_attn_args, o_sh);
  F(shrimp_ray_attn_args, o_sn); F(shrimp_ray_attn_args, B); F(shrimp_ray_attn_args, H);
  F(shrimp_ray_attn_args, N); F(shrimp_ray_attn_args, D); F(shrimp_ray_attn_args, blockers);
  Z(shrimp_raytap_args);
  F(shrimp_raytap_args, x); F(shrimp_raytap_args, x_sb); F(shrimp_raytap_args, x_sn);
  F(shrimp_raytap_args, gather_idx); F(shrimp_raytap_args, g_sb); F(shrimp_raytap_args, g_sn);
  F(shrimp_raytap_args, mask); F(shrimp_raytap_args, packed_w); F(shrimp_raytap_args, bias);
  F(shrimp_raytap_args, ln_w); F(shrimp_raytap_args, ln_b); F(shrimp_raytap_args, ray_idx);
  F(shrimp_raytap_args, r_sb); F(shrimp_raytap_args, r_sn); F(shrimp_raytap_args, reach);
  F(shrimp_raytap_args, re_sb); F(shrimp_raytap_args, re_sn); F(shrimp_raytap_args, alpha);
  F(shrimp_raytap_args, eps); F(shrimp_raytap_args, relu); F(shrimp_raytap_args, corb);
  F(shrimp_raytap_args, out); F(shrimp_raytap_args, o_sb); F(shrimp_raytap_args, o_sn);
  F(shrimp_raytap_args, B); F(shrimp_raytap_args, N); F(shrimp_raytap_args, C);
  F(shrimp_raytap_args, Cout);
  return 0;
}
