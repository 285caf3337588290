"""CPU oracle of the block-FP8 path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
the product path in hf_kernels_helion_amd never touches it.

Parity status of each function (how it is pinned; see tests/test_oracle.py):
  e4m3fn_from_f32 / e4m3fn_to_f32 : pinned against torch's float8_e4m3fn cast
      over every bf16 bit pattern and a dense fp32 sweep, and the 256-code
      decode table (tests/golden/e4m3fn_cast_table.npz).
  act_quant        : pinned by closed forms (s == amax/448, amax element ->
      +-448), a brute-force nearest-grid-point search, scale invariance under
      powers of two, and the non-finite policy cases.
  act_quant_f32    : (fp32 values; fp16 inputs widened) bit-equal to act_quant
      on bf16-representable values, and pinned by torch's CPU evaluation of
      the contract (fp32 division, float8_e4m3fn cast) on random fp32 and
      fp16 groups, the s == amax/448 closed form and the non-finite policy.
  block_gemm       : pinned against float64 brute force, exact small-integer
      cases (As = Bs = 1), one-hot rows, power-of-two row scaling and K-block
      permutation invariance.
  dequant_matmul   : pinned against torch's CPU fp64 matmul of the dequantised
      operands.
  silu_and_mul     : pinned against torch.nn.functional.silu in fp32 with the
      reference's rounding points, to 1 bf16 ulp.
  silu_and_mul_typed : (fp32/fp16/bf16 in and out) pinned against torch's CPU
      evaluation of act.py's expression for every dtype pair (within one ulp
      of the output type, mostly bit-equal) and bit-equal to silu_and_mul on
      bf16.
  quant_weight_block : pinned by the same closed forms as act_quant applied per
      128x128 block, torch's float8_e4m3fn cast of W / Bs on finite blocks, and
      the non-finite policy cases (NaN block, +-inf block, subnormal block).
"""
from .oracle import (  # noqa: F401
    load,
    bf16_bits,
    e4m3fn_from_f32,
    e4m3fn_to_f32,
    act_quant,
    act_quant_f32,
    block_gemm,
    dequant_matmul,
    silu_and_mul,
    silu_and_mul_typed,
    quant_weight_block,
)
