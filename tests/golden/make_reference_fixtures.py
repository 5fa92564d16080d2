"""Writes tests/golden/reference_fixtures.npz from the reference's own code, imported from
/root/reference on the CPU (the tests that run on the GPU never need the reference itself, only these vectors).
It pins what no closed form or library routine pins:

  init_*    sha256 of every tensor of the reference's seed-0 model (train/val/eggroll.py:38-53
            make_model('cpu', 0), fp32 bytes in state_dict order)
  fwd_*     GPT.forward mean cross-entropy (utils/model.py:193-209; flex_attention run by Inductor on the
            CPU, fp32) on two fixed sequences, at the seed-0 init and with lm_head scaled x30
  pop_*     population_loss (train/val/eggroll.py:66-103, fp32 on the CPU) for 4 members x 256 tokens with
            rank-1 noise on every one of the 60 parameters (the reference requires all), lm_head x30

Run: python tests/golden/make_reference_fixtures.py   (about a minute: Inductor compiles flex on the CPU)
"""
import hashlib
import importlib.util
import sys

# importing the reference must not write bytecode caches into its (read-only) tree
sys.dont_write_bytecode = True
from pathlib import Path

import numpy as np
import torch

REF = Path('/root/reference')
OUT = Path(__file__).resolve().with_name('reference_fixtures.npz')


POP_MEMBERS, POP_TOKENS, POP_SIGMA, POP_SEED = 4, 256, 0.01, 4321


def population_inputs(shapes):
    """The population case's inputs, regenerated from a CPU generator (so the fixture stores only outputs):
    per-direction noise rows [2, out + in] (matrices) or [2, n] (vectors) in `shapes` order (the
    reference's named_parameters order), the +-sigma signs and the 257 token ids."""
    g = torch.Generator().manual_seed(POP_SEED)
    flat = {n: torch.randn(POP_MEMBERS // 2, sum(s), generator=g) for n, s in shapes.items()}
    sign = torch.tensor([POP_SIGMA, -POP_SIGMA]).repeat(POP_MEMBERS // 2)
    idx = torch.randint(0, 4096, (POP_TOKENS + 1,), generator=g)
    return flat, sign, idx


def load_reference():
    sys.path.insert(0, str(REF))
    spec = importlib.util.spec_from_file_location('reference_eggroll', REF / 'train' / 'val' / 'eggroll.py')
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    eg = load_reference()
    model = eg.make_model('cpu', 0)
    state = model.state_dict()
    names = list(state.keys())
    hashes = [hashlib.sha256(state[n].detach().float().contiguous().numpy().tobytes()).hexdigest() for n in names]

    g = torch.Generator().manual_seed(1234)
    seqs = torch.randint(0, 4096, (2, 257), generator=g)
    with torch.no_grad():
        x, y = seqs[:, :-1].contiguous(), seqs[:, 1:].contiguous()
        fwd_init = model(x, y).item()
        model.lm_head.weight.mul_(30.0)
        fwd_head30 = model(x, y).item()

    # population_loss with noise on all parameters (the head stays x30)
    params = dict(model.named_parameters())
    flat, sign, idx = population_inputs({n: tuple(p.shape) for n, p in params.items()})
    noise = {n: (tuple(t.repeat_interleave(2, 0) for t in rows.split(list(params[n].shape), dim=1))
                 if params[n].dim() == 2 else rows.repeat_interleave(2, 0)) for n, rows in flat.items()}
    with torch.no_grad():
        pop = eg.population_loss(model, params, noise, sign, idx[:-1], idx[1:])

    arrays = dict(
        init_names=np.array(names), init_sha256=np.array(hashes),
        fwd_seqs=seqs.numpy(), fwd_loss_init=np.float32(fwd_init), fwd_loss_head30=np.float32(fwd_head30),
        pop_idx=idx.numpy(), pop_sign=sign.numpy(), pop_losses=pop.numpy().astype(np.float32),
    )
    np.savez_compressed(OUT, **arrays)
    print(f'wrote {OUT}: fwd {fwd_init:.6f} / {fwd_head30:.6f}, population {pop.tolist()}')


if __name__ == '__main__':
    main()
