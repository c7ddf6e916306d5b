"""The language-model shell against the reference's (tests/golden/lm_small.pt,
written by make_lm_golden.py from model.py:179-216 with the pure-torch layer).

CPU only: the oracle shell reproduces the reference's initialisation bit for
bit (state dicts equal), its logits and loss, and its FP32 gradients; the
product's ``BDMLanguageModel`` builds the identical state dict on the CPU
(construction only, no compute)."""

import os

import pytest
import torch

from conftest import ROOT
from oracle import bdm_oracle as O

GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'lm_small.pt')


@pytest.fixture(scope='module')
def golden():
    return torch.load(GOLDEN, weights_only=True)


def memory_config(golden):
    from bdm_amd import BSDMConfig
    dim, j, s, k, v, h = golden['geometry'][:6].tolist()
    return BSDMConfig(dim=dim, bank_count=j, bank_size=s, selected_banks=k, value_width=v, num_heads=h)


def oracle_model(golden):
    vocab, layers, multiple, seed = golden['geometry'][6:].tolist()
    return O.OracleLanguageModel(memory_config(golden), vocab_size=vocab, layers=layers, multiple_of=multiple,
                                 seed=seed)


def test_oracle_init_matches_reference(golden):
    model = oracle_model(golden)
    state = model.state_dict()
    assert list(state) == list(golden['state'])
    for key, value in golden['state'].items():
        assert torch.equal(state[key], value), key


def test_product_init_matches_reference(golden):
    from bdm_amd.lm import BDMLanguageModel, LanguageModelConfig
    vocab, layers, multiple, seed = golden['geometry'][6:].tolist()
    config = LanguageModelConfig(memory=memory_config(golden), vocab_size=vocab, layers=layers,
                                 ffn_multiple_of=multiple, seed=seed)
    state = BDMLanguageModel(config).state_dict()
    assert list(state) == list(golden['state'])
    for key, value in golden['state'].items():
        assert torch.equal(state[key], value), key


def test_oracle_forward_loss_and_gradients(golden):
    model = oracle_model(golden)
    logits = model(golden['tokens'])
    assert torch.allclose(logits, golden['logits'], rtol=1e-5, atol=1e-6)
    loss = model(golden['tokens'], golden['target'])
    assert float(loss.detach()) == pytest.approx(float(golden['loss']), rel=1e-6)
    loss.backward()
    params = dict(model.named_parameters())
    for name, grad in golden['grads'].items():
        ref = grad.abs().max()
        assert float((params[name].grad - grad).abs().max() / ref) < 1e-5, name


def test_oracle_prefill_then_step_equals_forward(golden):
    """Stateful inference through the oracle shell (FP32 caches): prefill of a
    prefix then one step per token gives the logits the full forward gives
    at those positions; the recurrence's state rounding points are the only
    difference (training rounds the state to BF16 every 16 events), so FP32
    training state is used for the forward here."""
    import dataclasses
    model = oracle_model(golden)
    for block in model.layers:
        block.attention.config = dataclasses.replace(block.attention.config, training_state_dtype='float32')
    tokens = golden['tokens']
    with torch.no_grad():
        full = model(tokens)
        fp32 = [block.attention.create_state(tokens.shape[0], torch.float32) for block in model.layers]
        logits, caches = model.prefill(tokens[:, :12], fp32)
        assert torch.allclose(logits[:, 0], full[:, 11], rtol=1e-4, atol=1e-5)
        for t in range(12, 16):
            logits, caches = model.step(tokens[:, t:t + 1], caches)
            assert torch.allclose(logits[:, 0], full[:, t], rtol=1e-4, atol=1e-5), t
