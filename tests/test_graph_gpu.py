"""HIP graph capture of the inference calls (torch.cuda.CUDAGraph): the library launches only
kernels on the caller's stream (no host synchronisation, no memset, no allocation of its own),
and the binding allocates outputs and workspaces through torch, which a capture serves from the
graph's pool. Each graph is replayed several times, with new inputs copied in and eager work
and synchronisations between the replays, and every replay is compared with an eager call on
the same inputs: bitwise, since the graph runs the same kernels on the same data.

Covered: flash_attn_func on a grid that takes the key split (two kernels and a workspace) and on
one that does not, and flash_attn_with_kvcache decode over a paged cache with several splits
(scratch) and with cache lengths changed between replays."""
import pytest

pytestmark = pytest.mark.gpu


def _replays(capture_fn, refresh, eager_fn, n=3):
    """capture_fn() -> output tensor, captured once; refresh(i) writes new inputs in place;
    eager_fn() -> the same call run eagerly. Returns the max |difference| over n replays."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):          # warm (plans, allocator) outside the capture
            capture_fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = capture_fn()
    worst = 0.0
    for i in range(n):
        refresh(i)
        torch.cuda.synchronize()
        junk = torch.randn(1 << 20, device="cuda").sum()   # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        ref = eager_fn()
        torch.cuda.synchronize()
        worst = max(worst, (out.float() - ref.float()).abs().max().item())
        del junk
    return worst


@pytest.mark.parametrize("shape", [(1, 2048, 4, 128, True), (2, 512, 32, 64, False)],
                         ids=["key split", "one workgroup per query tile"])
def test_flash_attn_func_graph_replays(shape):
    import torch

    from fable_attn.flash_attn_interface import flash_attn_func
    B, S, H, D, causal = shape
    print(f"[graph] flash_attn_func {shape}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(1)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=torch.float16, generator=g) for _ in range(3))
    split = _fwd_split_bytes(q, k, causal) > 0
    assert split == (shape[0] == 1), "the first shape must take the key split, the second not"

    def refresh(i):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, device="cuda", dtype=t.dtype, generator=g))

    call = lambda: flash_attn_func(q, k, v, causal=causal)
    assert _replays(call, refresh, call) == 0.0


def _lib_strides(t):
    from fable_attn import _lib
    return _lib.Strides(t.stride(0), t.stride(2), t.stride(1))


def _fwd_split_bytes(q, k, causal):
    from fable_attn import _C, _lib
    B, S, H, D = q.shape
    s = _lib_strides
    p = _lib.FableFwdParams(None, None, None, None, None, s(q), s(k), s(k), s(q), S, k.shape[1], D, H,
                            H // k.shape[2], D ** -0.5, 0.0, -1, -1, None, int(causal), 0.0, 0, None, None,
                            B, 0, None, None, H * S, S)
    return _C._L.fable_attn_fwd_ws_bytes(p, 0)


def test_kvcache_decode_graph_replays():
    import torch

    from fable_attn.flash_attn_interface import flash_attn_with_kvcache
    print("[graph] flash_attn_with_kvcache paged decode", flush=True)
    B, Hq, Hk, D, page, nb = 4, 16, 4, 128, 256, 64
    g = torch.Generator(device="cuda").manual_seed(2)
    kc = torch.randn(nb, page, Hk, D, device="cuda", dtype=torch.bfloat16, generator=g)
    vc = torch.randn(nb, page, Hk, D, device="cuda", dtype=torch.bfloat16, generator=g)
    bt = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).view(B, nb // B).int().cuda()
    lens = torch.tensor([4000, 1, 2500, 4096], dtype=torch.int32, device="cuda")
    q = torch.randn(B, 1, Hq, D, device="cuda", dtype=torch.bfloat16, generator=g)

    def refresh(i):
        q.copy_(torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=g))
        lens.copy_(torch.tensor([4000 - 900 * i, 1 + 700 * i, 2500, 4096 - i], dtype=torch.int32))

    from fable_attn import _C
    assert _C.num_splits(B, 1, Hq, Hq // Hk, bt.shape[1] * page, 0) > 1, "the decode must split"
    call = lambda: flash_attn_with_kvcache(q, kc, vc, cache_seqlens=lens, block_table=bt, causal=True)
    assert _replays(call, refresh, call) == 0.0
