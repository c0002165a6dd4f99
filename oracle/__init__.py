"""CPU oracle for the decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import this
package: only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, and only as the checker / the timed CPU
baseline.  The GPU library fails loudly when its HIP build is missing; it
never falls back to anything in here.

Modules
-------
ref     -- torch (CPU, fp32 math) restatement of rmsnorm_tkg, router_topk,
           moe_tkg, attention_block_tkg and the Qwen3-MoE fused layer flow,
           including the reference's bf16 rounding points.
mx      -- numpy restatement of OCP-MX (E8M0 block scale + E4M3 / E2M1
           element) quantisation, bit-level.

Parity pinning (what checks each function; see tests/test_oracle_*.py):
  rmsnorm_tkg          HF Qwen3MoeRMSNorm (fp32), closed forms, padding law
  router_topk          HF Qwen3MoeTopKRouter (fp32), brute force on tiny E,
                       invariants (row sums, K non-zeros)
  moe_tkg              HF Qwen3MoeExperts (fp32), one-hot == dense SwiGLU MLP
  attention (generic)  torch SDPA (fp32), S=1 / uniform-score closed forms
  rope                 HF apply_rotary_pos_emb, position 0 identity
  qwen layer / step    HF Qwen3MoeDecoderLayer (fp32) via golden fixtures
  mx                   OCP MX v1.0 spec: exact KATs (powers of two, every
                       representable E4M3 / E2M1 value round-trips), every
                       E4M3 code and RNE+saturation against torch's
                       float8_e4m3fn, E2M1 rounding by brute force
  moe_tkg_mx           = moe_tkg on the dequantised weights up to the
                       activation quantisation (bounded), exact when the
                       activations are MX-representable
"""
