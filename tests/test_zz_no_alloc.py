"""wc_verify_chain_greedy_static -- the greedy chain verify with its scratch in a
static device array instead of a caller workspace -- returns the verdict of
wc_verify_chain_greedy bit for bit: two calls in a row through the C ABI, the
second over fewer rows and a narrower vocabulary (what the first left in the
scratch must not leak into it), then a row count beyond what the scratch holds
is rejected."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref_and_static(cuda, rows, vocab, n_agree, seed):
    from woodcock_amd import _lib
    from woodcock_amd.runtime import new_verdict, ptr, stream_ptr, workspace

    g = torch.Generator(device=cuda).manual_seed(seed)
    logits = torch.randn(rows, vocab, generator=g, device=cuda) * 3
    drafts = torch.randint(0, vocab, (rows - 1,), generator=g, device=cuda, dtype=torch.int32)
    for i in range(min(n_agree, rows - 1)):  # planted agreement: a = n_agree
        logits[i, int(drafts[i])] = 1e4
    if n_agree < rows - 1:
        logits[n_agree, int(drafts[n_agree])] = -1e4
    want, got = new_verdict(cuda), new_verdict(cuda)
    _lib.call("wc_verify_chain_greedy", ptr(logits), rows, vocab, logits.stride(0), ptr(drafts), ptr(want),
              ptr(workspace(cuda)), stream_ptr())
    _lib.call("wc_verify_chain_greedy_static", ptr(logits), rows, vocab, logits.stride(0), ptr(drafts), ptr(got),
              stream_ptr())
    torch.cuda.synchronize()
    return want, got


def test_static_scratch_verify_equals_workspace_verify(cuda):
    from woodcock_amd import _lib

    want, got = _ref_and_static(cuda, 9, 151936, 5, seed=1)
    assert torch.equal(got, want)
    assert int(got[_lib.V_N_ACCEPTED]) == 5 and int(got[_lib.V_STATUS]) == 0
    want, got = _ref_and_static(cuda, 4, 5000, 1, seed=2)  # smaller, right after
    assert torch.equal(got, want)
    assert int(got[_lib.V_N_ACCEPTED]) == 1


def test_static_scratch_rejects_too_many_rows(cuda):
    from woodcock_amd import _lib
    from woodcock_amd.runtime import new_verdict, ptr, stream_ptr

    rows = _lib.WC_MAX_NODES + 1
    logits = torch.zeros(rows, 128, device=cuda)
    drafts = torch.zeros(rows - 1, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("wc_verify_chain_greedy_static", ptr(logits), rows, 128, 128, ptr(drafts), ptr(new_verdict(cuda)),
                  stream_ptr())
