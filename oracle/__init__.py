"""CPU oracle for the causal-chunk attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, in fp32 (and float64 for brute-force pinning) on the CPU, the
reference's own PyTorch semantics of the hot path:

  * Wan RoPE tables and the causal 3-D grid (wan/modules/model.py:47-53, 480-487;
    wan/modules/model_fast.py:878-979)
  * RMSNorm of q/k, both as the nn.Module (model.py:126-142) and as the fused
    q/k post-processing kernel sequence (kernels/qk_post.py:88-141), token rows and the
    head-major d-major ``_t`` layout with q's scale folded into cos/sin (qk_post.py:216-306)
  * windowed exact attention, the SDPA fallback of attention() (attention.py:1127-1143)
    with the KV window mask of model_fast.py:2538-2545, looped per head and query
    block so no [H, Lq, Lk] score tensor is ever materialised
  * the unnormalised-partial / log-sum-exp merge contract (attention.py:617-645, 963-990)
  * chunked KV-cache routing (wan/modules/chunked_kv_cache.py:36-76)
  * the fp8-e4m3 KV quantiser (no reference counterpart; the algorithm is defined here)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker. The product path (lbw_amd) never imports it and has
no CPU fallback: it raises when the HIP library is missing.
"""
from .wan_ref import *  # noqa: F401,F403
