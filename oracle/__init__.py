"""TEST INFRASTRUCTURE ONLY — CPU oracle of the MoE feed-forward hot path.

This package is the checker, never the product: only tests/, the smoke() of
__graft_entry__ and the cpu_baseline leg of bench.py may import it.  The
product path (kolmogorov-moe-architecture_amd/kmoe) runs on the HIP kernels
only and fails loudly without them.

moe_oracle.py   numpy restatement of the reference algorithm, function by
                function, each citing the reference file:line it follows.
torch_port.py   op-for-op torch-CPU restatement of the reference's default
                PyTorch path (padded bmm experts); the timed CPU baseline.

Pinning (how each oracle function is checked independently, tests/test_oracle.py):
  router_logits      fp64 per-token brute-force loops; torch nn.Sequential(Linear,SiLU,Linear)
  topk_select        brute-force sort on (-logit, index); torch.topk on tie-free rows
  softmax/aux_losses closed forms: uniform logits -> z = (ln E)^2, LB = 1 for balanced
                     counts with uniform probabilities; brute-force loops
  dispatch           numpy/torch stable argsort + bincount (library routines); brute force
  swiglu_rows        fp64 per-token brute force
  plain_rows         fp64 per-token, per-unit loops; torch_port's padded bmm with w3 None
  combine            brute-force per-token sums
  ec_select          brute-force sort on (-logit, index); torch.topk on tie-free columns
  mod_select         brute-force sort; torch.topk + sort on tie-free rows
  f32_to_e4m3        torch.float8_e4m3fn cast (library routine) on saturated inputs,
                     exhaustively over every code and every rounding midpoint
  quant_rows         round trip: amax element -> exactly +-448, error <= 2^-4 of the amax
  bf16_round         torch fp32 -> bfloat16 cast (library routine) on random values,
                     exact ties, overflow to inf, subnormals, +-0, +-inf; NaN stays NaN
  quant_weight_cols  torch restatement (per-(expert, output column) amax over K,
                     float8_e4m3fn cast); per-column brute force (amax element exact,
                     error <= 2^-4 of the column amax), columns of 1e3x / 1e-3x scale
  swiglu_rows_fp8    torch fake-quant restatement (bf16 and e4m3 library casts);
                     fp64 per-token brute force at a tiny shape
  mod_logits         torch nn.Linear(d, 1, bias=False) in fp64; brute force
  torch_port vs moe_oracle at small shapes (two independent restatements)
  moe_loss_tc_routed forward = torch_port.moe_layer_tc at its own routing; its
                     autograd gradients = finite differences (gradcheck, fp64)
  rms_norm           torch.nn.functional.rms_norm (library routine); unit mean square at
                     weight 1, eps 0; invariance under scaling of x; per-element brute force
  ffn_block_tc       h + torch_port.moe_layer_tc(F.rms_norm(h)) (independent restatement)
Every function above has at least one check that does not restate its own formula.
"""
