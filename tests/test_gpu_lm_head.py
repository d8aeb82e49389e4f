"""GPU parity of the fused decode-step output projection (mi_lm_head): final
RMSNorm + lm_head GEMV + greedy argmax, against the CPU oracle (oracle.quant's
rmsnorm, then an fp32 matmul of the dtype-rounded rows) and against the
engine's unfused GPU chain (RMSNorm kernel + torch Linear).

Bars: logits within 2e-2 of the logit scale of the fp32 oracle (bf16/fp16
outputs, as the other bf16 projections); the greedy tokens are exactly
torch.argmax of the kernel's own logits (first index among equal maxima), so
the token check is bit-exact.
"""
import pytest
import torch

from helpers import max_abs, randn
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _close(a, b, tol):
    scale = float(b.float().abs().max()) + 1e-6
    assert max_abs(a, b) < tol * scale, (max_abs(a, b), scale)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,N", [(1, 512, 1000), (8, 2048, 128256), (16, 2048, 5003),
                                   (3, 4096, 777), (8, 3072, 40000), (5, 1024, 16)])
@pytest.mark.parametrize("norm", [True, False])
def test_logits_and_greedy_tokens(dev, dtype, M, K, N, norm):
    from src.lm_head import lm_head
    from src.rms_norm import rmsnorm_triton
    x = randn((M, K), 1, dtype, dev, scale=2.0)
    w = randn((N, K), 2, dtype, dev, scale=K ** -0.5)
    nw = (1.0 + 0.1 * randn((K,), 3, torch.float32)).to(dtype).to(dev) if norm else None
    y, tok = lm_head(x, w, nw, 1e-5, greedy=True)
    assert y.shape == (M, N) and y.dtype == dtype and tok.shape == (M,)
    a = oq.rmsnorm(x, nw, 1e-5) if norm else x.cpu()
    ref = a.float() @ w.cpu().float().t()
    _close(y, ref, 2e-2)
    # the unfused GPU chain: RMSNorm kernel, then the library GEMM
    un = torch.nn.functional.linear(rmsnorm_triton(x, nw, 1e-5) if norm else x, w)
    _close(y, un, 1e-2)
    # greedy tokens: bit-exact argmax of the returned logits
    assert torch.equal(tok.cpu(), torch.argmax(y.float(), dim=-1).cpu())
    # logits-only call writes the same logits
    assert torch.equal(lm_head(x, w, nw, 1e-5), y)


def test_ties_keep_the_first_index(dev):
    from src.lm_head import lm_head
    M, K, N = 4, 512, 3000
    x = randn((M, K), 5, torch.bfloat16, dev)
    w = randn((N, K), 6, torch.bfloat16, dev, scale=0.01)
    # rows 7, 1500 and 2999 all equal x-aligned direction: the largest logits,
    # equal in every row; the first of them must win (torch.argmax rule)
    v = x[0].float() / x[0].float().norm()
    for n in (2999, 7, 1500):
        w[n] = (v * 4).to(torch.bfloat16)
    y, tok = lm_head(x[:1].expand(M, K).contiguous(), w, greedy=True)
    assert float(y[0, 7]) == float(y[0, 1500]) == float(y[0, 2999])
    assert tok.tolist() == [7] * M


def test_ragged_tail_and_strided_rows(dev):
    from src.lm_head import lm_head
    M, K, N = 6, 1024, 1003            # last tile has 11 valid rows
    base = randn((M, K + 64), 7, torch.bfloat16, dev)
    x = base[:, :K]                    # row stride K + 64 (16-byte aligned)
    w = randn((N, K), 8, torch.bfloat16, dev, scale=K ** -0.5)
    y, tok = lm_head(x, w, greedy=True)
    ref = x.cpu().float() @ w.cpu().float().t()
    _close(y, ref, 2e-2)
    assert torch.equal(tok.cpu(), torch.argmax(y.float(), dim=-1).cpu())


def test_unsupported_shapes_are_rejected(dev):
    from src import lm_head as lh
    w = randn((100, 512), 9, torch.bfloat16, dev)
    assert not lh.supported(17, 512, w)
    assert not lh.supported(4, 500, w)
    with pytest.raises(NotImplementedError):
        lh.lm_head(randn((17, 512), 10, torch.bfloat16, dev), w)
    with pytest.raises(TypeError):
        lh.lm_head(randn((2, 512), 10, torch.float16, dev), w)


def test_graph_runner_greedy_loop(dev):
    """decode_greedy feeds its device tokens back without a host round trip;
    the tokens equal the argmax of the same step's logits."""
    from src.config import ModelArgs
    from src.cuda_graph import CUDAGraphDecodeRunner
    from src.kv_cache import KVCache
    from src.model_quantized import build_random_quantized
    args = ModelArgs(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, vocab_size=4096,
                     hidden_dim=1024, max_batch_size=4, max_seq_len=256, device=str(dev))
    model = build_random_quantized(args, seed=0, device=str(dev))
    kv = KVCache(args, dtype=torch.bfloat16)
    runner = CUDAGraphDecodeRunner(model, args, kv, str(dev), batch_size=4, greedy=True)
    tok = torch.randint(0, args.vocab_size, (4, 1), generator=torch.Generator().manual_seed(0)).to(dev)
    for pos in range(3):
        nxt = runner.decode_greedy(tok, pos)
        logits = runner.static_logits
        assert torch.equal(nxt.reshape(-1).cpu(),
                           torch.argmax(logits.reshape(4, -1).float(), dim=-1).cpu())
        tok = nxt.clone()
