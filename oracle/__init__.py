"""CPU restatement of nanochat's fp8-KV decode path: TEST INFRASTRUCTURE ONLY.

This package is the checker, never the thing measured or shipped. Only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s `cpu_baseline` leg may import it. The product path (`nanochat_amd`) never imports it and has no CPU
fallback: it fails loudly when its HIP library is missing.

Modules:
  golden   numpy restatement: rotary tables, QK-norm + RoPE row math, bf16/fp8 rounding, per-(token, kv head)
           fp8 quantisation, the paged cache layout, append, gather, position rows, decode and chunked-prefill
           attention (fp64).
  sampling the token choice: Philox4x32-10, Gumbel-max, nucleus, masks and the commit.
  model    the decoder on the CPU (torch bf16 GEMMs over golden's append and attention): the end-to-end checker
           and the config 5 CPU baseline.

Parity pins (tests/test_oracle.py): every function is checked against a closed form, an exhaustive table, torch's
own float8_e4m3fn / bfloat16 casts (library routines), or brute force on tiny inputs. The reference ships no
golden vectors for this path and its CUDA sources cannot be built here (sm_90a inline PTX, nvcc absent), so
`oracle/_ref` stays empty. The one thing no check can pin is the reference's exact rounding of QK-norm: its CUDA
path uses rsqrtf and a lane-local butterfly (model/kernels/qk_row.cuh:25-30), its torch path
torch.rsqrt(mean) (inference/modeling_nanochat.py:41-45). This oracle fixes one documented rule instead
(golden.qk_norm_rope) and is pinned against the closed forms; parity with the reference's own bits for that one
rounding choice is "unpinned".
"""
