"""CPU oracle for the Shrimp forward hot path — TEST INFRASTRUCTURE ONLY.

A plain restatement of the reference's algorithm (numpy for the integer
tables, eager torch on the CPU for the floating-point forward), each function
citing the reference file:line it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker / the timed CPU baseline: the shipped
``shrimp`` package never imports anything from here.

How each part is pinned (so a dropped term, wrong sign or transposed operand
fails a check), see tests/test_oracle_*.py:
  tables.cell_lut / pair_rows   golden pair tensor from the reference, the
                                bijection / ring / far-row invariants of
                                tests/test_shrimp_geometry.py, brute force
  tables.ray_index              golden index from the reference join
                                (hexfield_eq/_triton_ray.py:221-281), brute
                                force dictionary join on tiny boards
  forward.hex_conv              dense F.conv2d on an embedded 41x41 grid (fp64),
                                as tests/test_shrimp_model.py:81-136
  forward.raytap_conv           reduces to hex_conv when only the distance-1
                                slots carry weight; brute-force loop
  forward.attention             torch scaled_dot_product_attention on the same
                                materialised bias (test_shrimp_model.py:65-78)
  forward.forward_policy_value  golden outputs of the reference ShrimpNet
                                (cfg0 and cfg4 architectures, fp32)
  decode.*                      golden decode / evaluator replies of the
                                reference; closed forms (uniform logits, one-hot)
"""
