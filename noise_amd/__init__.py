"""noise_amd: the MI355X (gfx950) population-forward hot path of pculaf/noise.

Hand-written HIP kernels behind the C ABI of include/noise_amd.h (libnoise_amd.so), with Python
mirrors of the reference's call sites: utils/model.py `attention`, train/val/eggroll.py `lowrank`,
`lowrank_embed`, `population_loss` and `Eggroll` noise bookkeeping, train/val/run.py `head_loss`.
"""
from . import _lib  # noqa: F401
from . import ops  # noqa: F401,E402  (registers the torch.ops.noise_amd drop-ins)
