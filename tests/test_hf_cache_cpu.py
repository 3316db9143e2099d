"""CPU tests of the host logic of atflash.hf.PagedCache (no kernel calls):
length bookkeeping under HF's crop contract (transformers' DynamicLayer.crop:
a non-negative argument is the number of tokens to keep, a negative one the
number to drop from the end), the capacity check and the page-table layout."""
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import Qwen2Config  # noqa: E402

from atflash import hf  # noqa: E402


def _cache(capacity=100, batch=2):
    cfg = Qwen2Config(vocab_size=64, hidden_size=512, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    return hf.PagedCache(cfg, batch, capacity, device="cpu")


def test_page_table_gives_each_sequence_its_own_pages():
    c = _cache(capacity=100, batch=2)
    assert c.pages_per_seq == 7  # ceil(100 / 16)
    assert c.page_table.tolist() == [list(range(7)), list(range(7, 14))]
    assert len(c.layers) == 2
    assert tuple(c.layers[0].k.shape) == (14, 2, 16, 16, 8)
    assert tuple(c.layers[0].v.shape) == (14, 2, 128, 16)


@pytest.mark.parametrize("arg,expect", [(30, 30), (0, 0), (50, 40), (40, 40), (-5, 35), (-40, 0), (-100, 0)])
def test_crop_follows_the_hf_contract(arg, expect):
    lyr = _cache().layers[0]
    lyr.length, lyr.prev_length, lyr.last_key = 40, 32, object()
    lyr.crop(arg)
    assert lyr.length == expect
    assert lyr.prev_length == min(32, expect)
    if expect < 40:
        assert lyr.last_key is None  # the hook must not take a stale key as this layer's


def test_update_refuses_more_tokens_than_the_capacity():
    lyr = _cache(capacity=20, batch=1).layers[0]
    lyr.length = 15
    k = torch.zeros((1, 2, 6, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="holds 20 tokens"):
        lyr.update(k, k)
    bad = torch.zeros((1, 3, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="do not fit"):
        lyr.update(bad, bad)
