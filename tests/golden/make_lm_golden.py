"""Writes ``lm_small.pt``: a two-layer language model of the reference's
shell (``implementation/bdm/model.py:143-216`` with ``backend='reference'``,
the pure-torch layer) as plain tensors.

Run once in the build container, which holds the read-only reference at
/root/reference; the GPU box never runs this.  Stored: the seeded state dict
(pins the shell's initialisation order and seeds), fixed tokens and targets,
the FP32 logits, the cross-entropy loss, and FP32 gradients of the loss for
the embedding, the output head and the first block's feed-forward.

Usage:  python tests/golden/make_lm_golden.py [/root/reference/implementation]
"""

from __future__ import annotations

import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GRADS = ('tok_embeddings.weight', 'output.weight', 'layers.0.feed_forward.w1.weight',
         'layers.0.feed_forward.w2.weight', 'layers.1.ffn_norm.weight', 'norm.weight')


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    from bsdm import BSDMConfig, BSDMLanguageModel, LanguageModelConfig  # noqa: E402

    memory = BSDMConfig(dim=32, bank_count=16, bank_size=8, selected_banks=4, value_width=32, num_heads=2)
    config = LanguageModelConfig(memory=memory, vocab_size=64, layers=2, ffn_multiple_of=32, seed=1)
    model = BSDMLanguageModel(config, backend='reference')
    gen = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, 64, (2, 20), generator=gen)
    target = torch.randint(0, 64, (2, 20), generator=gen)
    logits = model(tokens)
    loss = model(tokens, target)
    loss.backward()
    params = dict(model.named_parameters())
    out = dict(
        state={k: v.detach().clone() for k, v in model.state_dict().items()},
        tokens=tokens, target=target, logits=logits.detach(), loss=loss.detach(),
        grads={name: params[name].grad.detach().clone() for name in GRADS},
        geometry=torch.tensor([32, 16, 8, 4, 32, 2, 64, 2, 32, 1]),
    )
    torch.save(out, os.path.join(HERE, 'lm_small.pt'))
    print('wrote', os.path.join(HERE, 'lm_small.pt'))


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference/implementation')
