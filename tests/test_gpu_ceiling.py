"""GPU check of bench.py's ceiling copy (include/xt_ceiling.h): the bytes it
moves are the ones it claims, for the one-pass shapes of both size classes
(two vectors a thread up to 32 MiB, eight beyond), including a last
workgroup that is only partly inside the array."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 12582912 + 16, (32 << 20), (32 << 20) + 16, (40 << 20) + 48])
def test_ceiling_copy_moves_every_byte(cuda, nbytes):
    import torch

    import bench

    lib = bench._ceiling_lib()
    print(f"[gpu] ceiling copy {nbytes} B", flush=True)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=cuda)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=cuda)
    dst[nbytes:] = 7  # past the end: must stay untouched
    stream = torch.cuda.current_stream(cuda)
    assert lib.xt_ceiling_copy(src.data_ptr(), dst.data_ptr(), nbytes, stream.cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 7).all())
