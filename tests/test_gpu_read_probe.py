"""GPU: the HBM read probes bench.py reports ceilings with (mnb_stream_read,
mnb_stream_read_grid) read every byte of the buffer exactly once: each
wavefront folds the 32-bit words it loads with XOR into its output word, so
the XOR of all output words equals the XOR of all words of the buffer (a
byte read twice or skipped changes it; reads past the end return zeros)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [
    (31498240, None), (31498240, (224, 512)),  # c2's bytes: default grid, GemvFragKernel's grid
    (4096, None), (4096, (256, 1024)),          # fewer bytes than wavefronts x 1 KiB
    (10518528 + 16, (64, 448)),                 # shares not a multiple of 8 KiB
])
def test_probe_reads_every_word_once(pkg, cuda, nbytes, grid):
    import torch
    print(f"case read probe bytes={nbytes} grid={grid}", flush=True)
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).to(cuda)
    words = 2048 if grid is None else grid[0] * grid[1] // 64
    out = torch.full((words,), -1, dtype=torch.int32, device=cuda)
    L = pkg.library()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    if grid is None:
        assert L.mnb_stream_read(P(buf), nbytes, P(out), words, st) == 0
    else:
        assert L.mnb_stream_read_grid(P(buf), nbytes, P(out), words, grid[0], grid[1], st) == 0
    torch.cuda.synchronize()
    folded = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    assert folded == np.bitwise_xor.reduce(host)
