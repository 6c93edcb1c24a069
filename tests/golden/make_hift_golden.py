"""Writes tests/golden/hift_reference_vectors.npz: outputs of the reference's own HiFT glue run on CPU.

The reference's ``engine/models/token2wav.py`` imports only torch and numpy at module level; its
``hift_forward_noise`` (f0 -> NSF source -> ``_hift_decode`` -> ``istft_overlap_add``), ``fade_in_out`` and
``chunk_noise_seed`` are run here on this repository's oracle HiFT object (which exposes the attribute names those
functions read), so the vectors pin the oracle's glue order (source construction, reflection-pad placement, source
cache overwrite, cross-fade) to the reference code.  Run in the build container only (the reference does not travel):

    python tests/golden/make_hift_golden.py /root/reference
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from engine.models import token2wav as ref  # the reference module (torch + numpy only)

    import t2w_amd  # noqa: F401
    from oracle import hift as oh
    from t2w_amd.config import HiFTConfig
    from t2w_amd.weights import init_hift

    h = oh.HiFT(init_hift(HiFTConfig(), seed=3))
    g = torch.Generator().manual_seed(11)
    T = 12
    mel = torch.randn(2, 80, T, generator=g) * 2 - 5
    cache_source = torch.randn(2, 1, 960, generator=g) * 0.01
    rand_ini, noise = oh.hift_noise(9, [3, 4], T * 480)
    with torch.no_grad():
        speech, source = ref.hift_forward_noise(h, mel, cache_source, rand_ini, noise)
    fade_a, fade_b = torch.randn(1, 8000, generator=g), torch.randn(1, 7000, generator=g)
    fade_out = ref.fade_in_out(fade_a, fade_b, torch.from_numpy(np.hamming(2 * ref.SOURCE_CACHE)))
    seed_args = np.array([[0, 0], [1, 1], [7, 3], [2 ** 62, 5]], dtype=np.int64)
    seeds = np.array([ref.chunk_noise_seed(int(a), int(b)) for a, b in seed_args], dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "hift_reference_vectors.npz"), mel=mel.numpy(), cache_source=cache_source.numpy(),
                        rand_ini=rand_ini.numpy(), noise=noise.contiguous().numpy(), speech=speech.numpy(), source=source.numpy(),
                        fade_a=fade_a.numpy(), fade_b=fade_b.numpy(), fade_out=fade_out.numpy(), seed_args=seed_args, seeds=seeds)
    print("wrote", os.path.join(HERE, "hift_reference_vectors.npz"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
