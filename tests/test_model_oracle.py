"""The oracle forward's fast form (x86-restated GEMMs, used by the 4B-architecture end-to-end test) equals its
scalar form on the synthetic qwen35 model: logits after a prefill and after decode steps, bit for bit (CPU only)."""
import numpy as np

from tests import gguf_ref as R
from tests.test_convert import synthetic_model
from tests.test_model_e2e import OracleModel, BITS, CTX, same


def test_oracle_forward_fast_equals_scalar():
    ref = R.convert_ref(synthetic_model(seed=7), BITS, CTX)
    slow, fast = OracleModel(ref), OracleModel(ref, fast=True)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, slow.vocab, 9).tolist()
    assert same(slow.forward(prompt), fast.forward(prompt))
    for _ in range(3):
        t = [int(rng.integers(0, slow.vocab))]
        assert same(slow.forward(t), fast.forward(t))
