"""Device-resident decode block tables (DecodeInputs): each step uploads only
the table entries a slot's device row lacks; after the update kernel every
live row's device table equals the batch's table exactly."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _batch(tables, rids, slots, epochs, lengths, bs):
    from tinyvllm.batch import PreparedBatch, StepMode
    from tinyvllm.request import SamplingParams

    n = len(tables)
    offsets = np.concatenate(([0], np.cumsum([len(t) for t in tables])))
    ids = np.concatenate([np.asarray(t, dtype=np.int64) for t in tables])
    pos = np.asarray(lengths) - 1
    slot_map = np.asarray([t[p // bs] * bs + p % bs for t, p in zip(tables, pos)])
    greedy = SamplingParams(max_new_tokens=100)
    return PreparedBatch(
        plan_id=0, mode=StepMode.DECODE_ONLY, input_ids=(1,) * n,
        positions=tuple(int(p) for p in pos), q_offsets=tuple(range(n + 1)),
        context_lens_before=tuple(int(p) for p in pos), query_lens=(1,) * n,
        context_lens_after=tuple(lengths), sample_token_indices=tuple(range(n)),
        sample_request_ids=tuple(rids), sampling_params=(greedy,) * n, kv_block_size=bs,
        kv_num_blocks=1000, kv_block_table_ids=ids,
        kv_block_table_offsets=tuple(int(o) for o in offsets), kv_slot_mapping=slot_map,
        request_ids=tuple(rids), request_slots=slots, kv_table_epochs=epochs)


def test_device_tables_track_growth_swaps_and_slot_reuse(device):
    from tinyvllm.runtime.inputs import DecodeInputs

    bs = 16
    inputs = DecodeInputs(max_num_seqs=4, max_model_len=256, block_size=bs, device=device)
    rng = np.random.default_rng(3)
    tables = {7: list(rng.permutation(1000)[:3]), 8: list(rng.permutation(1000)[:5]),
              9: list(rng.permutation(1000)[:1])}
    lengths = {7: 40, 8: 70, 9: 10}
    slot = {7: 2, 8: 0, 9: 3}
    epoch = {7: 1, 8: 2, 9: 3}
    uploads = []

    def step(rids):
        before = inputs.stats["table_entries"]
        batch = _batch([tables[r] for r in rids], rids, tuple(slot[r] for r in rids),
                       tuple(epoch[r] for r in rids), [lengths[r] for r in rids], bs)
        mi = inputs.prepare(batch, [0] * len(rids))
        inputs.apply_table_updates()
        torch.cuda.synchronize()
        uploads.append(inputs.stats["table_entries"] - before)
        table = inputs.table.cpu().numpy()
        offs = mi.kv.decode.block_table_offsets.cpu().numpy()
        for i, r in enumerate(rids):
            start = int(offs[i])
            assert start == slot[r] * inputs.pitch
            got = table[start:start + len(tables[r])]
            assert list(got) == [int(x) for x in tables[r]], r
        # Padding rows and the closing entry: one past the tables' end.
        full = inputs.d["offsets"].cpu().numpy()
        assert offs.size == len(rids) + 1
        assert (full[len(rids):] == inputs.table_capacity).all()

    step([7, 8, 9])                     # whole tables: 3 + 5 + 1
    assert uploads[-1] == 9
    step([7, 8, 9])                     # nothing changed
    assert uploads[-1] == 0
    tables[7].append(999)               # growth by one page
    lengths[7] = 49
    step([8, 7])                        # other order, row 9 absent
    assert uploads[-1] == 1
    tables[8][1] = 777                  # a prefix swap: new epoch, whole table
    epoch[8] = 10
    step([7, 8, 9])
    assert uploads[-1] == 5
    del tables[9]                       # request 9 ends; 11 takes its slot
    tables[11], lengths[11], slot[11], epoch[11] = [5, 6], 20, 3, 11
    step([7, 8, 11])
    assert uploads[-1] == 2
    batch = _batch([tables[7]], [7], None, None, [lengths[7]], bs)  # no slot record
    inputs.prepare(batch, [0])
    assert inputs.stats["table_entries"] - sum(uploads) == len(tables[7])
