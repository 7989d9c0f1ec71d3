"""The memory bank's public tensor API (backends/ctdg/runtime/memory.py:134-269)
against the oracle's MemoryO: write_mailbox (src pass then dst pass, one slot
per node and pass, the pointer advanced by the occurrence count),
_write_slots, _apply_memory_update, gather, read_mailbox, gather_mailbox and
read_mailbox_ts, bit-exact over several calls in a row with repeated nodes,
tied timestamps, an empty call, and edge features narrower or wider than the
mailbox's feature width."""
import pytest
import torch

import ctdg_oracle as co

pytestmark = pytest.mark.gpu


def _bank(gpu, N, D, K, F):
    from starry_unigraph.backends.ctdg.runtime.memory import CTDGMemoryBank
    return CTDGMemoryBank(num_nodes=N, hidden_dim=D, device=str(gpu), mailbox_slots=K, edge_feat_dim=F)


def _same_state(bank, ref, msg):
    st = bank.state
    for name, got, want in (("memory", st.memory, ref.memory), ("memory_ts", st.memory_ts, ref.memory_ts),
                            ("mailbox", st.mailbox, ref.mailbox), ("mailbox_ts", st.mailbox_ts, ref.mailbox_ts),
                            ("next_mail_pos", st.next_mail_pos.long(), ref.next_mail_pos)):
        assert torch.equal(got.cpu(), want), f"{msg}: {name}"


@pytest.mark.parametrize("K,ef_width", [(1, 6), (3, 6), (3, 4), (2, 9)])
def test_memory_bank_api_matches_oracle(gpu, K, ef_width):
    N, D, F = 40, 8, 6
    bank, ref = _bank(gpu, N, D, K, F), co.MemoryO(N, D, K, F)
    gen = torch.Generator().manual_seed(K * 10 + ef_width)
    v0, m0 = bank.mailbox_version, bank.memory_version
    for call, B in enumerate([25, 0, 60, 17, 33]):
        src = torch.randint(0, N, (B,), generator=gen)
        dst = torch.randint(0, N, (B,), generator=gen)
        # tied timestamps on purpose: integers from a narrow range
        ts = torch.randint(0, 6, (B,), generator=gen).float() + 10.0 * call
        smem = torch.randn(B, D, generator=gen)
        dmem = torch.randn(B, D, generator=gen)
        ef = torch.randn(B, ef_width, generator=gen)
        bank.write_mailbox(src.to(gpu), dst.to(gpu), smem.to(gpu), dmem.to(gpu), ef.to(gpu), ts.to(gpu))
        ref.write_mailbox(src, dst, smem, dmem, ef, ts)
        _same_state(bank, ref, f"write_mailbox call {call}")
        # a memory update of distinct nodes with per-row times
        ids = torch.randperm(N, generator=gen)[:max(1, B // 3)]
        vals = torch.randn(ids.numel(), D, generator=gen)
        uts = torch.rand(ids.numel(), generator=gen) * 100
        bank._apply_memory_update(ids.to(gpu), vals.to(gpu), uts.to(gpu))
        ref.apply_memory_update(ids, vals, uts)
        _same_state(bank, ref, f"_apply_memory_update call {call}")
    assert bank.mailbox_version == v0 + 5 and bank.memory_version == m0 + 5
    q = torch.randint(0, N, (50,), generator=gen)
    qg = q.to(gpu)
    assert torch.equal(bank.gather(qg).cpu(), ref.memory[q])
    assert torch.equal(bank.read_mailbox(qg).cpu(), ref.mailbox[q])
    assert torch.equal(bank.gather_mailbox(qg).cpu(), ref.mailbox[q][:, 0, :])
    assert torch.equal(bank.read_mailbox_ts(qg).cpu(), ref.mailbox_ts[q])
    assert bank.read_mailbox(qg).shape == (50, K, 2 * D + F)
    # ids given on the host are read from the bank's device too
    assert torch.equal(bank.gather(q).cpu(), ref.memory[q])


def test_write_slots_matches_serial_rules(gpu):
    """_write_slots of one pass against the serial loop of the write rules
    (every event of a node writes the slot read once; the last in stable
    time order survives; the pointer advances by the count)."""
    N, D, K, F = 12, 4, 3, 2
    bank, ref = _bank(gpu, N, D, K, F), co.MemoryO(N, D, K, F)
    gen = torch.Generator().manual_seed(9)
    for call in range(4):
        B = 30
        ids = torch.randint(0, N, (B,), generator=gen)
        vals = torch.randn(B, 2 * D + F, generator=gen)
        ts = torch.randint(0, 4, (B,), generator=gen).float()
        bank._write_slots(ids.to(gpu), vals.to(gpu), ts.to(gpu))
        co.write_slots_serial(ref, ids, vals, ts)
        _same_state(bank, ref, f"_write_slots call {call}")
