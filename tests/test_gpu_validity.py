"""Emission scan (alignment.cu:893-917) against a torch reduction: one record
per bad position class (unaligned head, unrolled body, remainder, tail) so
every loop of the scan kernel sees a rejected value."""
import pytest
import torch

from fast_forced_aligner import emission_validity

pytestmark = pytest.mark.gpu


def _expected(records):
    return [not bool((torch.isnan(r) | torch.isposinf(r)).any()) for r in records]


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
@pytest.mark.parametrize("frames,vocab", [(1, 1), (3, 5), (257, 31), (2305, 33), (20001, 40)])
def test_scan_matches_torch_at_every_position_class(offset, frames, vocab):
    n = frames * vocab
    generator = torch.Generator(device="cuda").manual_seed(n + offset)
    positions = sorted({0, 1, 2, 3, n // 3, n // 2, n - 4, n - 3, n - 2, n - 1} & set(range(n)))
    records = []
    for k, pos in enumerate(positions):
        storage = torch.randn(n + offset, generator=generator, device="cuda")
        record = storage[offset:].view(frames, vocab)  # contiguous view, 4*offset bytes off alignment
        record[pos // vocab, pos % vocab] = (torch.nan, torch.inf, -torch.inf)[k % 3]
        records.append(record)
    records.append(torch.randn(frames, vocab, generator=generator, device="cuda"))
    assert emission_validity(records).tolist() == _expected(records)


def test_scan_many_records():
    generator = torch.Generator(device="cuda").manual_seed(5)
    records = [torch.randn(int(t), 7, generator=generator, device="cuda")
               for t in torch.randint(1, 400, (3000,), generator=generator, device="cuda").tolist()]
    for i in range(0, len(records), 7):
        records[i][-1, 0] = torch.inf if i % 2 else torch.nan
    assert emission_validity(records).tolist() == _expected(records)
