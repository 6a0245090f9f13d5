"""recap_refresh_capture_noalloc, the capture entry point that allocates nothing (its
validation partials live in a static device array), against recap_refresh_capture with a
caller workspace on identical inputs: refinement, log-mass and validation sums bit for bit,
on two calls in a row, the second smaller, and the size limit enforced on the host."""

import pytest
import torch

from gpu_util import capture_inputs
from recap_amd import _lib
from recap_amd import kernels as K

pytestmark = pytest.mark.gpu


def _run(x, cuda, validate, noalloc):
    banks, rows, d = x["oh"].shape[0], x["rows"], x["oh"].shape[-1]
    det = (x["old"][0].clone() if validate
           else torch.zeros(banks, rows, d, dtype=torch.float16)).to(cuda)
    dl = (x["old"][1].clone() if validate else torch.zeros(banks, rows)).to(cuda)
    glref = x["old"][2].to(cuda) if validate else None
    center = x["old"][3].to(cuda) if validate else None
    args = (x["of"].to(cuda), x["lf"].reshape(banks, -1).contiguous().to(cuda),
            x["oh"].to(cuda), x["lh"].to(cuda), x["go"].to(cuda), x["gl"].to(cuda),
            torch.as_tensor(x["rowmap"]).to(cuda), K.Geometry(x["n"], x["n_video"]), det, dl)
    if noalloc:
        stats = torch.full((2,), float("nan"), device=cuda) if validate else None
        K.refresh_capture_noalloc(*args, stats, glref=glref, center=center)
    else:
        stats = K.refresh_capture(*args, glref=glref, center=center)
    torch.cuda.synchronize()
    return det.cpu(), dl.cpu(), None if stats is None else stats.cpu()


@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float16)])
def test_noalloc_capture_equals_workspace_capture(cuda, d, dtype):
    # two calls in a row on the shared scratch, the second with fewer banks and rows
    for banks, blocks, validate in [(4, 9, True), (2, 3, True), (3, 5, False)]:
        print(f"case d={d} {dtype} banks={banks} blocks={blocks} validate={validate}",
              flush=True)
        x = capture_inputs(d, dtype, False, seed=31 * banks + blocks, banks=banks,
                           blocks=blocks)
        want = _run(x, cuda, validate, noalloc=False)
        got = _run(x, cuda, validate, noalloc=True)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        if validate:
            assert torch.equal(got[2], want[2]), (got[2], want[2])
            print(f"  validation sums {got[2].tolist()}", flush=True)


def test_noalloc_capture_rejects_sizes_beyond_its_scratch(cuda):
    """More banks than the 4 MiB scratch holds partial pairs for: rejected on the host,
    before any launch (no device buffer is touched)."""
    d, n_video = 128, 128 * 64
    per_bank = int(_lib.load().recap_capture_partials(1, d, n_video))
    banks = _lib.CAPTURE_NOALLOC_MAX_PAIRS // per_bank + 1
    x = torch.zeros(16, dtype=torch.bfloat16, device=cuda)
    f = torch.zeros(16, device=cuda)
    with pytest.raises(ValueError, match="static scratch holds"):
        _lib.call("recap_refresh_capture_noalloc", x.data_ptr(), _lib.RECAP_BF16, 1, banks, d,
                  banks * n_video * d, n_video * d, d, f.data_ptr(), x.data_ptr(), f.data_ptr(),
                  x.data_ptr(), f.data_ptr(), f.data_ptr(), n_video, n_video, x.data_ptr(),
                  f.data_ptr(), f.data_ptr(), f.data_ptr(), f.data_ptr(), None)
