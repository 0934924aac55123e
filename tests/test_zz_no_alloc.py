"""ferry_layout_noalloc (the layout with its workspace in a static device buffer) against
ferry_layout, both through the C ABI: two calls in a row with the same output buffers, the
second with fewer tokens (one-block and three-kernel layouts), bit-exact on every output;
sizes beyond the static buffer are rejected before any launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc():
    from ferry_amd._lib import lib
    return lib().ferry_layout_noalloc


def _outputs(T, k, E, device):
    return dict(send_ids=torch.full((T, k), -7, dtype=torch.int64, device=device),
                w_sorted=torch.full((T, k), 3, dtype=torch.int16, device=device),
                starts=torch.full((E + 1,), -7, dtype=torch.int64, device=device),
                rows=torch.full((T * k,), -7, dtype=torch.int64, device=device),
                cols=torch.full((T * k,), -7, dtype=torch.int64, device=device),
                pair_pos=torch.full((T * k,), -7, dtype=torch.int32, device=device))


def _ptrs(o):
    return [o[n].data_ptr() for n in ('send_ids', 'w_sorted', 'starts', 'rows', 'cols', 'pair_pos')]


@pytest.mark.parametrize('sizes', [(70000, 3000, 5), (900, 17)])
def test_layout_noalloc_matches_layout(device, sizes):
    from ferry_amd._lib import last_error, lib
    from ferry_amd import expert_ops as ops
    E, k = 128, 8
    fn = _noalloc()
    stream = torch.cuda.current_stream().cuda_stream
    a = _outputs(sizes[0], k, E, device)       # shared by every no-alloc call
    for T in sizes:
        print(f'layout_noalloc: T={T} E={E} k={k}', flush=True)
        g = torch.Generator().manual_seed(T)
        sel = torch.argsort(torch.rand((T, E), generator=g), dim=1)[:, :k].contiguous().to(device)
        w = torch.randn((T, k), generator=g).to(torch.bfloat16).to(device)
        ref = ops.layout(sel, w, E)
        assert ops.layout_errors(ref) == 0
        o = dict(send_ids=a['send_ids'][:T], w_sorted=a['w_sorted'][:T], starts=a['starts'],
                 rows=a['rows'][:T * k], cols=a['cols'][:T * k], pair_pos=a['pair_pos'][:T * k])
        rc = fn(sel.data_ptr(), w.data_ptr(), T, k, E, *_ptrs(o), stream)
        assert rc == 0, last_error()
        torch.cuda.synchronize()
        assert torch.equal(o['send_ids'], ref.send_ids)
        assert torch.equal(o['w_sorted'], ref.w_sorted.view(torch.int16))
        assert torch.equal(o['starts'], ref.starts)
        assert torch.equal(o['rows'], ref.rows) and torch.equal(o['cols'], ref.cols)
        assert torch.equal(o['pair_pos'], ref.pair_pos)
    # a layout past the static buffer is rejected without a launch
    big = 600 * 1024
    rc = fn(None, None, big, k, E, *([None] * 6), stream)
    assert rc != 0 and 'scratch' in last_error()
    assert lib().ferry_layout_workspace_bytes(big, k, E) > 256 + 128 * 512 * 4
