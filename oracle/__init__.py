"""CPU oracle for the joyomni_ops hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes for each op
of deploy/joyomni_ops (jd-opensource/JoyAI-Video-Edit), each function citing
the reference file:line it follows. It is the checker, never the product:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and the shipped package (joyai-video-edit_amd/joyomni_ops) never
does.

Modules:
  ops.py      torch-on-CPU restatements of every op (fp32 arithmetic).
  fp8_ref.c   independent C restatement of the FP8 e4m3fn encoding and of the
              per-token quantization rule (brute-force nearest-code search),
              built into oracle/_build/libfp8ref.so by oracle/build.py.
  fp8ref.py   ctypes loader for fp8_ref.c.

How each function is pinned (there are no golden vectors in the reference;
its tests only print fp32-formula diffs):
  per_token_quant_fp8   C brute-force encoder (all 256 codes) + hand-derived
                        known answers (zero row, NaN, Inf, ties, saturation).
  rmsnorm               torch.nn.functional.rms_norm (library routine) and
                        the unit-RMS invariant.
  norm_scale_shift      torch.nn.functional.layer_norm / rms_norm + closed
                        form of the modulation on hand-picked rows.
  qk_norm_rope_table    complex multiplication (torch.polar / view_as_complex)
                        and norm preservation; identity rotation.
  rope_grid_tables      float64 closed form of the angles, cos^2+sin^2=1,
                        angle addition for the source-id composition.
  add_layernorm_*       composition of torch.addcmul and F.layer_norm.
  rmsnorm_quant_fp8     composition of the rmsnorm restatement and the C
                        per-token / per-block quantizer.
  norm_scale_shift_quant_fp8  composition of residual_add / norm_scale_shift
                        and per_token_quant_fp8 (each pinned above).
  apply_rotary_emb      identity and quarter-turn tables (exact), complex
                        multiplication in float64, a planted sign slip.
  commit_kv             apply_rotary_emb per layer + copies (pool regions
                        outside the segment unchanged).
  fp8_scaled_mm         exact integer matmul (int64 on the fp8 values times
                        2^9) equals the float64 accumulation; decoding of all
                        256 codes against the C encoder's table; the
                        epilogue order against a hand-checked row.
"""
