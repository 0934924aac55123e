"""DeepSeek-V2-Lite-shaped layer on the HIP path: shared experts, the fused bf16 addition in the
combine, and the single-layer parity case (T = 256, 64 experts top-6, intermediate 1408, plus
the 2 shared experts, all experts resident): routing indices and permutation bit-exact, output
within rel 2e-2 / abs 1e-2 of the reference's result and of an fp64 SwiGLU."""
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.experts import (deepseek_layer_ref, moe_fp64, reduce_partials_ref, shared_mlp_fp64,
                            shared_mlp_ref)
from oracle.layout import layout_closed_form
from oracle.router import deepseek_router

pytestmark = pytest.mark.gpu


def _ops():
    from ferry_amd import expert_ops
    return expert_ops


@pytest.mark.parametrize('T,H,I', [
    (16, 2048, 2816),     # decode: skinny kernels
    (256, 2048, 2816),    # the single-layer case: tiled kernels
    (97, 512, 384),       # ragged: one partial M tile
    (0, 256, 128),        # empty
])
def test_shared_expert_vs_hf_mlp(device, T, H, I):
    from ferry_amd import workloads
    ops = _ops()
    row = workloads.shared_rows(1, H, I, seed=3, device=device)[0]
    g = torch.Generator().manual_seed(T + 5)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    shared = ops.SharedExpert(row, H, I)
    out = shared(x.to(device))
    torch.cuda.synchronize()
    assert out.shape == (T, H) and out.dtype == torch.bfloat16
    if T == 0:
        return
    row_c = row.cpu()
    ref = shared_mlp_ref(row_c, x, H, I)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    exact = shared_mlp_fp64(row_c, x, H, I).float()
    torch.testing.assert_close(out.cpu().float(), exact, rtol=2e-2, atol=1e-2)


def test_combine_add_is_bf16_addition(device):
    """bf16(fp32(bf16(sum_j part)) + fp32(addend)): bit-exact with torch's bf16 add on the CPU."""
    ops = _ops()
    T, k, H = 300, 6, 2048
    g = torch.Generator().manual_seed(9)
    part = torch.randn((T * k, H), generator=g).to(torch.bfloat16)
    addend = (torch.randn((T, H), generator=g) * 3).to(torch.bfloat16)
    perm = torch.randperm(T * k, generator=g)
    pair_pos = perm.to(torch.int32)
    out = ops.combine(part.to(device), T, k, H, pair_pos=pair_pos.to(device), addend=addend.to(device))
    routed = reduce_partials_ref([part[perm[j::k]] for j in range(k)],
                                 [torch.arange(T)] * k, T, H)
    assert torch.equal(out.cpu(), routed + addend)
    # without addend the plain combine is unchanged
    plain = ops.combine(part.to(device), T, k, H, pair_pos=pair_pos.to(device))
    assert torch.equal(plain.cpu(), routed)


@pytest.mark.parametrize('pack', [False, True])
def test_deepseek_layer_t256_all_resident(device, pack):
    """One DeepSeek-V2-Lite MoE layer, 256 tokens, every expert resident (64 slots); with packed
    fetches (17.3 MB rows of 2816-wide experts) the output equals the raw fetches' bit for bit."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import deepseek_moe
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.DEEPSEEK_LAYER_T256
    spec = w.spec
    E, k, H, I, T = spec.experts, spec.topk, spec.hidden, spec.intermediate, w.tokens
    pool = workloads.make_pool(spec, 1, seed=w.seed)
    gate = workloads.router_gates(spec, 1, seed=w.seed, device=device)[0]
    srow = workloads.shared_rows(1, H, w.shared_intermediate, seed=w.seed, device=device)[0]
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, E), pack=pack)
    shared = ops.SharedExpert(srow, H, w.shared_intermediate)
    out, logits = deepseek_moe(rt, 0, x, gate, k, shared=shared)
    torch.cuda.synchronize()
    if pack:
        assert rt.packed.ratio > 1.3
        raw_rt = OffloadRuntime(spec, pool, [w.cache_slots], 'ferry', Topology.uniform(1, E))
        raw_out, _ = deepseek_moe(raw_rt, 0, x, gate, k, shared=shared)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), raw_out.cpu())
        raw_rt.close()
    # routing: the oracle on the identical fp32 logits (the GEMM is not part of the parity claim)
    lg = logits.cpu()
    w_ref, sel_ref, _ = deepseek_router(lg, k)
    wts, sel = ops.router_topk(logits, k, renorm=False, sorted=False)
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(wts.cpu(), w_ref)   # the kernel's fp32 softmax is torch's, bit for bit
    # permutation
    lay = ops.layout(sel, wts, E)
    ref_lay = layout_closed_form(sel_ref.numpy(), E, w_ref.float().numpy())
    for key in ('send_ids', 'starts', 'rows', 'cols'):
        assert np.array_equal(getattr(lay, key).cpu().numpy(), ref_lay[key]), key
    # every routed expert was fetched once into the empty cache, none evicted
    assert rt.h2d.copies == len(np.unique(sel_ref.numpy()))
    # output
    ref = deepseek_layer_ref(lambda e: pool[e], srow.cpu(), x.cpu(), sel_ref, w_ref, E, H, I,
                             w.shared_intermediate)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=2e-2, atol=1e-2)
    exact = (moe_fp64(lambda e: pool[e], x.cpu(), sel_ref, w_ref, H, I)
             + shared_mlp_fp64(srow.cpu(), x.cpu(), H, w.shared_intermediate)).float()
    torch.testing.assert_close(out.cpu().float(), exact, rtol=2e-2, atol=1e-2)
    rt.close()


def _tile_edge_tokens(starts, rows, rng, tile_m=256, block=32):
    """Per expert, tokens at the edges of its last (partial) M tile: the tile's first row, the
    first and last rows of its last 32-row block that holds rows (the kernel skips the blocks
    past the expert's end), two random rows of that tile; and the largest expert's first and
    last rows."""
    pick = set()
    counts = np.diff(starts)
    for e, n in enumerate(counts):
        if n == 0:
            continue
        a = int(starts[e])
        last0 = (n - 1) // tile_m * tile_m
        blk0 = max(last0, (n - 1) // block * block)
        for p in {last0, blk0, n - 1, *rng.integers(last0, n, 2).tolist()}:
            pick.add(int(rows[a + p]))
    big = int(np.argmax(counts))
    pick.update((int(rows[starts[big]]), int(rows[starts[big + 1] - 1])))
    return np.array(sorted(pick), np.int64)


def test_deepseek_prefill_t65536_sampled_tokens(device):
    """The DeepSeek-V2-Lite prefill layer at full size (65,536 tokens, top-6 of 64, plus the
    shared experts), experts resident.  Each token's output depends only on its own row and
    experts, so the oracle is evaluated exactly on a sample of tokens that covers every
    expert's partial last M tile and the largest expert's tail; routing and the layout are
    checked on every token."""
    from ferry_amd import expert_ops as ops
    from ferry_amd import workloads
    from ferry_amd.model import deepseek_moe
    from ferry_amd.quota import Topology
    from ferry_amd.runtime import OffloadRuntime
    w = workloads.DEEPSEEK_PREFILL_STACK
    spec = replace(w.spec, moe_layers=w.spec.moe_layers[:1])
    E, k, H, I, T = spec.experts, spec.topk, spec.hidden, spec.intermediate, w.tokens
    assert (E, k, H, I, T, w.shared_intermediate) == (64, 6, 2048, 1408, 65536, 2816)
    pool = workloads.make_pool(spec, 1, seed=w.seed)
    gate = workloads.router_gates(spec, 1, seed=w.seed, device=device)[0]
    srow = workloads.shared_rows(1, H, w.shared_intermediate, seed=w.seed, device=device)[0]
    x = workloads.hidden_states(T, H, seed=w.seed + 7, device=device)
    rt = OffloadRuntime(spec, pool, [E], 'ferry', Topology.uniform(1, E))
    shared = ops.SharedExpert(srow, H, w.shared_intermediate)
    out, logits = deepseek_moe(rt, 0, x, gate, k, shared=shared)
    torch.cuda.synchronize()
    lg = logits.cpu()
    w_ref, sel_ref, _ = deepseek_router(lg, k)
    wts, sel = ops.router_topk(logits, k, renorm=False, sorted=False)
    assert torch.equal(sel.cpu(), sel_ref)
    assert torch.equal(wts.cpu(), w_ref)
    lay = ops.layout(sel, wts, E)
    ref_lay = layout_closed_form(sel_ref.numpy(), E, w_ref.float().numpy())
    for key in ('starts', 'rows', 'cols'):
        assert np.array_equal(getattr(lay, key).cpu().numpy(), ref_lay[key]), key
    counts = np.diff(ref_lay['starts'])
    assert int(counts.max()) > 4096   # tiled MFMA path on the big experts
    # every expert's partial last M tile (its first row and its last 32-row block, where the
    # kernel skips the row blocks past the expert's end), the largest expert's first and last
    # rows, plus random tokens
    assert (counts % 256 != 0).sum() >= 56
    targeted = _tile_edge_tokens(ref_lay['starts'], ref_lay['rows'], np.random.default_rng(4))
    g = torch.Generator().manual_seed(4)
    pick = torch.unique(torch.cat([torch.from_numpy(targeted), torch.tensor([0, T - 1]),
                                   torch.randperm(T, generator=g)[:62]]))
    assert len(pick) >= 200
    xs = x.cpu()[pick]
    ref = deepseek_layer_ref(lambda e: pool[e], srow.cpu(), xs, sel_ref[pick], w_ref[pick], E, H, I,
                             w.shared_intermediate)
    torch.testing.assert_close(out.cpu()[pick].float(), ref.float(), rtol=2e-2, atol=1e-2)
    rt.close()
