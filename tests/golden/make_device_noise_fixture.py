"""Writes tests/golden/device_noise_fixture.npz on an MI355X: values of torch-ROCm's own device draws that the
reference makes (run there; torch's generator is the library routine being matched, the reference's code is
not involved):
  buffer_idx / buffer_val   elements of torch.randn(2**28, generator=Generator('cuda').manual_seed(0))
                            (eggroll.py:114) at fixed indices, fp32
  offsets                   Eggroll.offsets(step=0) for 512 pairs: one torch.randint(0, 2**28 - sum(shape),
                            (512,)) per parameter on Generator('cuda').manual_seed(0) (eggroll.py:117-120)
  cus, max_threads          the device properties the draw layout depends on
Run: python tests/golden/make_device_noise_fixture.py out.npz
"""
import sys

import numpy as np
import torch

sys.path.insert(0, str(__import__('pathlib').Path(__file__).resolve().parents[2]))


def main(out):
    from noise_amd.model import make_model
    dev = torch.device('cuda', 0)
    props = torch.cuda.get_device_properties(dev)
    buf = torch.randn(2 ** 28, device=dev, generator=torch.Generator(dev).manual_seed(0))
    g = torch.Generator().manual_seed(7)
    idx = torch.cat([torch.arange(0, 64), torch.arange(2 ** 19 - 8, 2 ** 19 + 8), torch.arange(2 ** 28 - 64, 2 ** 28),
                     torch.randint(0, 2 ** 28, (4096,), generator=g)])
    vals = buf[idx.to(dev)].cpu()
    params = dict(make_model('cpu', 0).named_parameters())
    og = torch.Generator(dev).manual_seed(0)
    offsets = np.stack([torch.randint(0, 2 ** 28 - sum(p.shape), (512,), device=dev, generator=og).cpu().numpy()
                        for p in params.values()])
    np.savez_compressed(out, buffer_idx=idx.numpy(), buffer_val=vals.numpy(), offsets=offsets,
                        param_names=np.array(list(params)), cus=np.int64(props.multi_processor_count),
                        max_threads=np.int64(props.max_threads_per_multi_processor))
    print(f'wrote {out}: {len(idx)} buffer elements, offsets {offsets.shape}, CUs {props.multi_processor_count}')


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else 'device_noise_fixture.npz')
