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
    kv = c.layers[0].kv
    assert tuple(kv.shape) == (14, 2, 2, 2048) and kv.is_contiguous()
    assert tuple(c.layers[0].k.shape) == (14, 2, 16, 16, 8)
    assert tuple(c.layers[0].v.shape) == (14, 2, 128, 16)
    # k and v are views of the K and V halves of each (page, kv head) block
    c.layers[0].k[3, 1, 2, 5, 6] = 1.0
    c.layers[0].v[4, 0, 100, 7] = 2.0
    flat = kv.view(-1)
    assert (flat == 1.0).nonzero().flatten().tolist() == [((3 * 2 + 1) * 2 + 1) * 2048 + (2 * 16 + 5) * 8 + 6]
    assert (flat == 2.0).nonzero().flatten().tolist() == [((4 * 2 + 0) * 2 + 0) * 2048 + 100 * 16 + 7]


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


def test_an_unread_update_blocks_the_next_one():
    """update() returns only the new tokens, so a layer whose update no hook
    call read (another attention implementation, or a copied key) refuses the
    next update instead of letting attention run on the chunk alone."""
    c = _cache(capacity=64, batch=1)
    lyr = c.layers[1]
    lyr.last_key = object()  # an update that the hook has not read
    k = torch.zeros((1, 2, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="not read by the atflash"):
        lyr.update(k, k)
    assert c.pending(1) and not c.pending(0)


def test_hook_refuses_a_copied_key_of_a_pending_layer():
    """The hook finds a PagedCache layer by the identity of the key tensor;
    when a layer at the module's index holds an unread update under another
    tensor (a copy), it raises rather than treating the copy as the history."""
    from atflash.model_tables import window_from_config
    c = _cache(capacity=64, batch=1)
    cfg = Qwen2Config(vocab_size=64, hidden_size=512, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, rope_theta=1e4, max_position_embeddings=64)
    hook = hf.WindowAttention(window_from_config(cfg, 2.0, 2.0, 64), "win", rope_at_load=False)
    key = torch.zeros((1, 2, 3, 128), dtype=torch.bfloat16)
    c.layers[0].last_key = key

    class M:
        layer_idx = 0
    assert hook._paged_layer(M(), key) is c.layers[0]
    with pytest.raises(RuntimeError, match="copy"):
        hook._paged_layer(M(), key.clone())
    M.layer_idx = 1  # no pending update at this index: a plain cache
    assert hook._paged_layer(M(), key.clone()) is None


def test_closed_cache_refuses_updates():
    c = _cache(capacity=64, batch=1)
    c.closed = True
    k = torch.zeros((1, 2, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="closed"):
        c.layers[0].update(k, k)


def test_rope_table_grows_geometrically():
    """On a plain cache the context grows by one token per decode step; the
    hook's (cos, sin) table is rebuilt only when it doubles."""
    from atflash.model_tables import window_from_config
    cfg = Qwen2Config(vocab_size=64, hidden_size=512, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, rope_theta=1e4, max_position_embeddings=4096)
    hook = hf.WindowAttention(window_from_config(cfg, 2.0, 2.0, 4096), "win", rope_at_load=True)
    sizes = []
    for n in range(100, 1200):
        t = hook.rope_table(n, "cpu")
        if not sizes or sizes[-1] != t.shape[0]:
            sizes.append(t.shape[0])
    assert sizes == [100, 200, 400, 800, 1600]
    assert hook.rope_table(4097, "cpu").shape[0] == 4097
