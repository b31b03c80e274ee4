"""CPU restatement of tiny-vLLM's decode-loop arithmetic -- TEST INFRASTRUCTURE ONLY.

This package is the parity oracle: plain torch-CPU (fp32 / fp64) and numpy
code that restates, function by function, what the reference computes on the
hot path. Each function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or the timed CPU
baseline), never as the product path. The product (``tiny-vllm_amd/tinyvllm``)
never imports this package and has no CPU fallback.

How each part is pinned (tests/test_oracle_*.py):
  paged_kv   -- closed form slot = table[p // bs] * bs + p % bs, brute force
                on tiny pools, bitwise row equality, -1 sentinel untouched.
  attention  -- float64 textbook loops on tiny inputs; torch SDPA (library);
                special cases L=1 -> V, identical keys -> mean(V), one
                dominant key -> its V, L=0 -> zeros.
  pointwise  -- transformers' Qwen3RMSNorm / apply_rotary_pos_emb (library)
                in fp32; closed forms (constant rows, unit weights, position 0
                -> identity rotation, g = 0 -> 0); rounding sequence checked
                against the stated expression on bf16 grids.
  sampling   -- torch.argmax (library); top-k = 1 and top-p -> 0+ reduce to
                argmax; kept set vs a float64 sort/cumsum restatement.
  model      -- transformers' Qwen3ForCausalLM with the same weights (fp32).
"""
