"""Host logic of the row -> state mapping (opendecider_amd.prefix_attn.group_rows), on the CPU: rows in any state
order, as the reference's `rows` gives them (src/opendecider/prefix_attn.py:103-117,152-154), become the grouped
layout the one-launch kernels take. Checked against a brute-force grouping."""
import pytest
import torch

from opendecider_amd.prefix_attn import group_rows


@pytest.mark.parametrize("seed,R,Ns", [(0, 1, 1), (1, 17, 4), (2, 64, 3), (3, 9, 12)])
def test_group_rows_matches_brute_force(seed, R, Ns):
    rs = torch.randint(0, Ns, (R,), generator=torch.Generator().manual_seed(seed))
    order, row_start, max_rows = group_rows(rs, Ns)
    want = [i for s in range(Ns) for i in range(R) if rs[i] == s]  # stable: rows of a state keep their order
    assert order.tolist() == want
    counts = [int((rs == s).sum()) for s in range(Ns)]
    assert row_start.dtype == torch.int32 and row_start.tolist() == [sum(counts[:s]) for s in range(Ns + 1)]
    assert max_rows == max(counts)
    # the same layout with max_rows given (no host read)
    o2, r2, m2 = group_rows(rs, Ns, max_rows=max(counts))
    assert torch.equal(o2, order) and torch.equal(r2, row_start) and m2 == max_rows


def test_group_rows_rejects_out_of_range_states():
    with pytest.raises(ValueError):
        group_rows(torch.tensor([0, 3]), 3)
    with pytest.raises(ValueError):
        group_rows(torch.tensor([-1, 0]), 3)
