"""The configs[4] training step: mask inputs from the device-resident span /
link lists (the configs[2] cross_doc_link generator), the metadata pass,
embedding, 12 layers (d 768, 12 heads of 64), RMSNorm, the tied linear head +
cross-entropy, backward and AdamW, on one packed row of T = 16384 random
token ids with random-init weights (model/modules/training_module.py:199-230
is the reference's step)."""
from __future__ import annotations

import torch

from . import synth
from .block_mask import build_block_mask
from .mask_creators import TokenLists
from .modules import TS2TSTrainingModule

T, VOCAB, LAYERS, DIM, HEADS = 16384, 50257, 12, 768, 12


def configs4_step(dev: torch.device, seed: int = 0):
    """Returns step() -> loss; step.model, step.row, step.T hold the pieces."""
    row = synth.config_rows(3, seed=seed)[0]
    lists = TokenLists(T, [row.spans], dev, words=row.words, link_rows=[row.link_rows])

    def creator(tokens, **kw):
        return build_block_mask(*lists.build())

    torch.manual_seed(seed)
    model = TS2TSTrainingModule.from_config(
        vocab_size=VOCAB, num_layers=LAYERS, model_dim=DIM, num_heads=HEADS, max_seq_len=T,
        dropout=0.0, drop_path_rate=0.0, block_mask_creator=creator).to(dev, torch.bfloat16)
    # the fused form: one kernel per parameter group step (-1.1 ms per step
    # against the foreach form at configs[4])
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)
    g = torch.Generator().manual_seed(seed)
    batch = {"tokens": torch.randint(0, VOCAB, (1, T + 1), generator=g).to(dev)}

    def step():
        loss = model(batch)
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    step.model, step.row, step.T = model, row, T
    return step
