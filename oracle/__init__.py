"""CPU oracle for the Qwen3 int8 decode hot path -- TEST INFRASTRUCTURE, not product code.

This package restates, in torch (fp32/fp64 on the CPU) and in C (``oracle/c/oracle.c``), the
reference's golden algorithms for every function on the path. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import or run it, and
only as the checker or the timed CPU baseline -- never as the thing measured or shipped. It does
not import ``iron_amd``; inputs are passed in as plain tensors.

Modules (each function cites the reference file:line it follows):
  numerics   bf16 rounding helpers
  gemv       int8 wire pack/unpack, bit-exact dequant, exact and premul GEMV goldens, quantizers
  norms      weighted RMSNorm (kernel numerics), two-halves RoPE, RoPE angle table
  attention  decode attention (exp2 fp32 golden, fp64 brute force), causal prefill attention
  blocks     fused QKV head and fused SwiGLU MLP goldens
  qwen3      the whole-model decode chain with bf16 operator boundaries
  provider   ``op.reference()`` provider for iron_amd operators (the reference/compare modes)
  cref       ctypes binding of the C restatement (liboracle.so)

Pinning: every function here is checked in ``tests/test_oracle_*.py`` against a closed form,
an invariant, an fp64 brute force or the independent C restatement, chosen so that a dropped
term, a wrong sign/index or a transposed operand fails. No function is "parity unpinned" except
the NPU intrinsic-level rounding of the reference kernels (aie_api exp2/tanh/invsqrt), which no
reference test pins either; the goldens here use exact fp32/fp64 math instead.
"""
