"""h3mi.prequant on the CPU: the offered quantization is returned only for
the offered tensor, unchanged, and only while it is offered."""
import torch

from h3mi import prequant


def test_offer_and_take():
    h = torch.randn(16, 32).to(torch.bfloat16)
    q, qs = torch.zeros(16, 32, dtype=torch.int8), torch.ones(16, 1)
    assert prequant.take(h) is None
    with prequant.offer(h, q, qs):
        got = prequant.take(h)
        assert got is not None and got[0] is q and got[1] is qs
        assert prequant.take(h.view(16, 32)) is not None       # same bytes, same layout
        assert prequant.take(h.clone()) is None                 # other storage
        assert prequant.take(h[:8]) is None                     # other shape
        assert prequant.take(h.t()) is None                     # other strides
        h.add_(1)                                               # changed in place
        assert prequant.take(h) is None
    assert prequant.take(h) is None                             # withdrawn


def test_offer_is_withdrawn_on_error():
    h = torch.randn(4, 8)
    try:
        with prequant.offer(h, None, None):
            raise RuntimeError("attention failed")
    except RuntimeError:
        pass
    assert prequant.take(h) is None
