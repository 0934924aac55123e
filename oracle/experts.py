"""Expert-FFN and combine oracle (test infrastructure).

``execute_experts_ref`` restates ferry/csrc/expert_ops.cpp:32-43 with expert_ops.cu:6-14 in
torch on the CPU (bf16 GEMMs with fp32 accumulation, bf16 rounding after each op);
``reduce_partials_ref`` restates expert_ops.cpp:76-83 (fp32 index_add_ in ascending group
order, then bf16).  ``moe_fp64`` is the high-precision SwiGLU used to pin both.
"""
import torch


def slot_weights(row, hidden, inter):
    part = hidden * inter
    gate = row[:part].view(inter, hidden)
    up = row[part:2 * part].view(inter, hidden)
    down = row[2 * part:].view(hidden, inter)
    return gate, up, down


def silu_mul_ref(g, u):
    """expert_ops.cu:6-14: bf16(g / (1 + exp(-g)) * u) computed in fp32."""
    g32, u32 = g.float(), u.float()
    return ((g32 / (1.0 + torch.exp(-g32))) * u32).to(torch.bfloat16)


def execute_experts_ref(weight_rows, x, routing_weights, rows, cols, hidden, inter):
    """Per group i: bf16 [n_i, H] = down(silu(x Wg^T) * (x Wu^T)) * w[rows, cols]."""
    outs = []
    for row, r, c in zip(weight_rows, rows, cols):
        gate, up, down = slot_weights(row, hidden, inter)
        xi = x.index_select(0, r)
        a = silu_mul_ref(xi @ gate.t(), xi @ up.t())
        y = a @ down.t()
        outs.append(y * routing_weights[r, c].unsqueeze(1))
    return outs


def reduce_partials_ref(parts, rows, received, hidden):
    partial = torch.zeros((received, hidden), dtype=torch.float32)
    for p, r in zip(parts, rows):
        partial.index_add_(0, r, p.float())
    return partial.to(torch.bfloat16)


def moe_layer_ref(weight_rows_of, x, selected, weights, experts, hidden, inter):
    """Reference layer at world = 1: layout, execute_experts in ascending e, reduce, bf16.

    ``weight_rows_of(e)`` returns the bf16 pool row of expert e.  ``weights`` are the bf16
    routing weights aligned with ``selected``.  Returns bf16 [T, H].
    """
    from .layout import layout_closed_form
    lay = layout_closed_form(selected.numpy(), experts, weights.float().numpy())
    w_sorted = torch.from_numpy(lay['w_sorted']).to(torch.bfloat16)
    groups = [e for e in range(experts) if lay['counts'][e] > 0]
    rows = [torch.from_numpy(lay['rows'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
    cols = [torch.from_numpy(lay['cols'][lay['starts'][e]:lay['starts'][e + 1]]) for e in groups]
    parts = execute_experts_ref([weight_rows_of(e) for e in groups], x, w_sorted, rows, cols,
                                hidden, inter)
    return reduce_partials_ref(parts, rows, x.shape[0], hidden)


def moe_fp64(weight_rows_of, x, selected, weights, hidden, inter):
    """fp64 SwiGLU MoE with no intermediate rounding (the numerical target of both paths)."""
    T, k = selected.shape
    out = torch.zeros((T, hidden), dtype=torch.float64)
    xd = x.double()
    for e in sorted(set(int(v) for v in selected.reshape(-1))):
        gate, up, down = (w.double() for w in slot_weights(weight_rows_of(e), hidden, inter))
        mask = (selected == e)
        tok = mask.any(1).nonzero().reshape(-1)
        w = (weights.double() * mask.double()).sum(1)[tok]
        g = xd[tok] @ gate.t()
        u = xd[tok] @ up.t()
        y = ((g / (1 + torch.exp(-g))) * u) @ down.t()
        out.index_add_(0, tok, y * w.unsqueeze(1))
    return out


def shared_mlp_ref(row, x, hidden, inter):
    """DeepSeek-V2 shared experts (HF DeepseekV2MLP, transformers modeling_deepseek_v2.py:140-153
    installed analogue): bf16 nn.Linear layers on the CPU, down(act(gate(x)) * up(x)) with the
    SiLU output and the product each rounded to bf16.  ``row`` is [gate | up | down]."""
    gate, up, down = slot_weights(row, hidden, inter)
    g = x @ gate.t()
    u = x @ up.t()
    a = torch.nn.functional.silu(g) * u
    return a @ down.t()


def shared_mlp_fp64(row, x, hidden, inter):
    gate, up, down = (w.double() for w in slot_weights(row, hidden, inter))
    g = x.double() @ gate.t()
    u = x.double() @ up.t()
    return ((g / (1 + torch.exp(-g))) * u) @ down.t()


def deepseek_layer_ref(weight_rows_of, shared_row, x, selected, weights, experts, hidden, inter,
                       shared_inter):
    """Routed experts through the reference's runtime order (moe_layer_ref), then the HF block's
    bf16 addition of the shared experts (modeling_deepseek_v2.py:136 installed analogue)."""
    routed = moe_layer_ref(weight_rows_of, x, selected, weights, experts, hidden, inter)
    return routed + shared_mlp_ref(shared_row, x, hidden, shared_inter)
