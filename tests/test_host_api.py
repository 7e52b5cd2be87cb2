"""Host-side contract of the drop-in wrappers (no GPU needed: these raise before any launch)."""
import pytest
import torch


def _qkv():
    q = torch.zeros(1, 4, 2, 128)
    return q, q.clone(), q.clone()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_attention_dtype_other_than_bf16_raises(dtype):
    """The reference computes in ``dtype`` (attention.py:1134-1141); these kernels compute in
    bf16, so asking for another dtype raises rather than silently returning bf16 accuracy."""
    from lbw_amd import attention, cross_attention, exact_attention, exact_attention_chunks
    q, k, v = _qkv()
    with pytest.raises(NotImplementedError, match="bfloat16"):
        attention(q, k, v, dtype=dtype)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        exact_attention(q, k, v, dtype=dtype)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        exact_attention_chunks(q, [k], [v], dtype=dtype)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        cross_attention(q, k, v, dtype=dtype)


def test_unsupported_options_raise():
    from lbw_amd import attention
    q, k, v = _qkv()
    with pytest.raises(NotImplementedError):
        attention(q, k, v, causal=True)
    with pytest.raises(NotImplementedError):
        attention(q, k, v, dropout_p=0.1)
    with pytest.raises(NotImplementedError):
        attention(q, k, v, window_size=(4, 4))


def test_cpu_tensors_are_rejected_loudly():
    """No CPU fallback: host tensors reach the device check and raise."""
    from lbw_amd import attention
    q, k, v = _qkv()
    with pytest.raises(RuntimeError, match="GPU tensor"):
        attention(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16))


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 (or a multi-rank launch) exits with status 2 and
    says so, before touching a device."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for argv, env in ((["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), *argv],
                           capture_output=True, text=True, timeout=120,
                           env={**os.environ, **env})
        assert r.returncode == 2, (argv, env, r.stdout, r.stderr)
        assert "one GPU" in r.stdout + r.stderr
