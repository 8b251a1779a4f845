"""Writes the golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/make_golden.py

Every expected value comes from the CPU oracle (oracle/) and is cross-checked
here against torch's eager flex_attention / create_block_mask on CPU with the
restated mask_mod before it is written.  Inputs are stored as bf16 bit
patterns (uint16) so the GPU tests feed the kernels exactly these values.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attn_oracle as ao  # noqa: E402
from oracle import mask_oracle as mo  # noqa: E402
from tagseq2tagseq_amd import synth  # noqa: E402
from tests.helpers import row_arrays  # noqa: E402

TABLES = ["kv_num_blocks", "kv_indices", "full_kv_num_blocks", "full_kv_indices",
          "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices"]


def _bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _from_bits(b: np.ndarray) -> np.ndarray:
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy().astype(np.float64)


def _check_against_torch(doc, qb, kb, ref):
    from torch.nn.attention.flex_attention import create_block_mask
    T = doc.shape[0]
    mod = mo.torch_mask_mod(torch.from_numpy(doc),
                            None if qb is None else torch.from_numpy(qb.view(np.int64)),
                            None if kb is None else torch.from_numpy(kb.view(np.int64)))
    bm = create_block_mask(mod, None, None, T, T, device="cpu")
    for name in TABLES:
        assert np.array_equal(ref[name], getattr(bm, name)[0, 0].numpy()), name
    return bm, mod


def mask_fixture(name, doc, qb, kb):
    ref = mo.block_mask_tables(doc, qb, kb)
    _check_against_torch(doc, qb, kb, ref)
    out = {"doc": doc, "tile_class": ref["partial"] + 2 * ref["full"]}
    if qb is not None:
        out["q_bits"] = qb
        out["kv_bits"] = kb
    out.update({n: ref[n] for n in TABLES})
    np.savez_compressed(os.path.join(HERE, f"mask_{name}.npz"), **out)


def attn_fixture(name, row, Hq, Hkv, D, seed):
    from torch.nn.attention.flex_attention import flex_attention
    doc, qb, kb = row_arrays(row)
    T = doc.shape[0]
    g = torch.Generator().manual_seed(seed)
    bits = {n: _bf16_bits(torch.randn(1, h, T, D, generator=g))
            for n, h in (("q", Hq), ("k", Hkv), ("v", Hkv), ("do", Hq))}
    q, k, v, do = (_from_bits(bits[n]) for n in ("q", "k", "v", "do"))
    dense = mo.dense_mask(doc, qb, kb)[None]
    o, lse = ao.attention_fwd(q, k, v, dense)
    dq, dk, dv = ao.attention_bwd(q, k, v, o, do, lse, dense)
    ref = mo.block_mask_tables(doc, qb, kb)
    bm, _ = _check_against_torch(doc, qb, kb, ref)
    qt, kt, vt = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    to, tl = flex_attention(qt, kt, vt, block_mask=bm, enable_gqa=Hq != Hkv, return_lse=True)
    to.backward(torch.from_numpy(do))
    for a, b in ((o, to), (lse, tl), (dq, qt.grad), (dk, kt.grad), (dv, vt.grad)):
        np.testing.assert_allclose(a, b.detach().numpy(), rtol=1e-9, atol=1e-9)
    # outputs as float16 (relative precision 5e-4, far inside the bf16 bound of 2e-2)
    out = dict(doc=doc, seed=np.int64(seed), **bits, lse=lse.astype(np.float32),
               o=o.astype(np.float16), dq=dq.astype(np.float16),
               dk=dk.astype(np.float16), dv=dv.astype(np.float16))
    if qb is not None:
        out["q_bits"] = qb
        out["kv_bits"] = kb
    np.savez_compressed(os.path.join(HERE, f"attn_{name}.npz"), **out)


def main():
    mask_fixture("config1_T1024", *row_arrays(synth.config_rows(1, seed=0)[0]))
    mask_fixture("config3_T4096", *row_arrays(synth.config_rows(3, seed=0, T=4096)[0]))
    mask_fixture("config4_T4096", *row_arrays(synth.config_rows(4, seed=0, T=4096)[0]))
    attn_fixture("cross_doc_link_T130_gqa", synth.linked_lognormal_docs(130, 20.0, 1.0, 60, 0.3, seed=5),
                 Hq=2, Hkv=1, D=64, seed=7)
    attn_fixture("doc_causal_T96_d128", synth.lognormal_docs(96, 20.0, 1.0, 60, seed=6),
                 Hq=1, Hkv=1, D=128, seed=8)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
