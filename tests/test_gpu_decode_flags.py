"""A decode step queued for one position range and replayed outside it is
caught on the device (asdsl_decode_token_upto, ASDSL_DECODE_FLAG_*): the
attention kernel sees the position at or past the range its grid was shaped
for (or outside the cache), zeroes its output, writes no K/V row and raises
a bit in the work buffer's flags word, which DecodeEngine reads at its sync
points.  Without the guard such a replay merged stale split partials of an
earlier step into the attention and produced wrong logits with no error."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture
def eng(gpu):
    from asdsl.engine import DecodeConfig, DecodeEngine

    e = DecodeEngine.synthetic(DecodeConfig(n_layers=1, vocab=2048, max_seq=1100), seed=3)
    e.prefill_kv_random(10, seed=4)
    e.token.fill_(7)
    return e


def _row_is_zero(eng, pos) -> bool:
    import torch

    L = eng.layers[0]
    return int(torch.count_nonzero(L["k_cache"][:, pos]).item()) == 0 and \
        int(torch.count_nonzero(L["v_cache"][:, pos]).item()) == 0


@pytest.mark.parametrize("start, past", [(10, 300), (600, 1050)])
def test_graph_replayed_past_its_range_raises(eng, start, past):
    """The short form (positions below 256: o_proj merges the splits) and the
    long form (below 1024: the combine kernel merges them), each replayed at
    a position its grid does not cover."""
    eng.pos.fill_(start)
    eng.capture()
    limit = eng._pos_limit(start)
    g = eng._graphs[limit]
    g.replay()
    eng.next_token()  # in range: no flag
    assert eng.device_flags() == 0
    assert not _row_is_zero(eng, start)
    eng.pos.fill_(past)  # behind the host's back, past the graph's range
    g.replay()
    with pytest.raises(RuntimeError, match="past the range"):
        eng.next_token()
    assert eng.device_flags() == 0  # cleared by the check
    assert int(eng.pos.item()) == past + 1  # the step still advanced token and position
    assert _row_is_zero(eng, past)  # and wrote no K/V row
    eng.pos.fill_(start + 1)  # back in range: the graph replays cleanly
    g.replay()
    eng.next_token()
    assert not _row_is_zero(eng, start + 1)


def test_position_outside_cache_raises(eng):
    """A replay that walks off the end of the cache raises FLAG_POS_RANGE."""
    eng.pos.fill_(eng.cfg.max_seq - 1)
    eng.capture()
    eng.step()
    eng.next_token()
    eng.step()  # position max_seq
    with pytest.raises(RuntimeError, match="outside the KV cache"):
        eng.next_token()
