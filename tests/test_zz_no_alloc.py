"""carat_hip_argmax_accept_noalloc (fixed per-device scratch, no allocation) against
carat_hip_argmax_accept (library workspace) through the C ABI: bit-identical predictions,
accepted lengths and next tokens on two calls in a row, the second smaller, with fp32 and bf16
logits in turn."""
import sys

import numpy as np
import pytest

from carat_amd import _lib
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run(torch, entry, logits, bf16, proposals, first, caps):
    rows, vocab = logits.shape
    requests, tokens = proposals.shape
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d_l = dev(logits.view(np.int16) if bf16 else logits)
    d_p, d_f = dev(proposals), dev(first)
    d_c = dev(caps) if caps is not None else None
    pred = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    acc = torch.full((requests,), -7, dtype=torch.int32, device="cuda")
    nxt = torch.full((requests,), -7, dtype=torch.int32, device="cuda")
    fn = getattr(_lib.lib(), entry)
    _lib.check(fn(None if bf16 else _lib.ptr(d_l), _lib.ptr(d_l) if bf16 else None, requests, tokens,
                  vocab, _lib.ptr(d_p), _lib.ptr(d_f), None if d_c is None else _lib.ptr(d_c),
                  _lib.ptr(pred), _lib.ptr(acc), _lib.ptr(nxt),
                  _lib.ptr(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    return pred.cpu().numpy(), acc.cpu().numpy(), nxt.cpu().numpy()


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_noalloc_argmax_accept_matches_workspace_entry(torch_cuda, bf16):
    torch = torch_cuda
    rng = np.random.default_rng(71 + bf16)
    # config 1 (24 x 5 x 262144), then a smaller ragged call that reuses the same scratch
    for requests, tokens, vocab in ((24, 5, 262144), (7, 3, 40000)):
        say(f"case: no-alloc argmax/accept {'bf16' if bf16 else 'f32'} {requests}x{tokens}x{vocab}")
        logits = rng.standard_normal((requests * tokens, vocab), dtype=np.float32)
        if bf16:
            logits = oracle.f32_to_bf16(logits)
        arg = (oracle.argmax_bf16_rows(logits) if bf16 else oracle.argmax_f32_rows_as_bf16(logits))
        arg = arg.reshape(requests, tokens)
        proposals = np.concatenate([rng.integers(0, vocab, (requests, 1)), arg[:, :-1]], 1).astype(np.int32)
        proposals[::2, tokens // 2] = (proposals[::2, tokens // 2] + 1) % vocab
        first = proposals[:, 0].copy()
        caps = rng.integers(0, tokens + 1, requests).astype(np.int32)
        want = run(torch, "carat_hip_argmax_accept", logits, bf16, proposals, first, caps)
        got = run(torch, "carat_hip_argmax_accept_noalloc", logits, bf16, proposals, first, caps)
        for a, b in zip(got, want):
            assert np.array_equal(a, b)
        exp_acc, exp_next = oracle.greedy_accept(proposals, first, arg, caps)
        assert np.array_equal(got[0], arg.reshape(-1))
        assert np.array_equal(got[1], exp_acc) and np.array_equal(got[2], exp_next)


def test_noalloc_argmax_accept_scratch_limit(torch_cuda):
    """The fixed scratch holds 65536 partial keys: 256 requests x 8 rows at vocabulary 262144 in
    fp32 (32 chunks of 8192 per row) fill it exactly and match the workspace entry point; one
    request more is rejected with the scratch error before anything runs (outputs untouched)."""
    torch = torch_cuda
    vocab, tokens = 262144, 8
    gen = torch.Generator(device="cuda").manual_seed(5)
    stream = _lib.ptr(torch.cuda.current_stream().cuda_stream)
    for requests in (256, 257):
        say(f"case: no-alloc scratch limit {requests}x{tokens}x{vocab} fp32")
        logits = torch.randn((requests * tokens, vocab), generator=gen, device="cuda")
        proposals = torch.randint(0, vocab, (requests, tokens), generator=gen, device="cuda",
                                  dtype=torch.int32)
        first = proposals[:, 0].contiguous()
        outs = {}
        for entry in ("carat_hip_argmax_accept", "carat_hip_argmax_accept_noalloc"):
            pred = torch.full((requests * tokens,), -7, dtype=torch.int32, device="cuda")
            acc = torch.full((requests,), -7, dtype=torch.int32, device="cuda")
            nxt = torch.full((requests,), -7, dtype=torch.int32, device="cuda")
            status = getattr(_lib.lib(), entry)(
                _lib.ptr(logits), None, requests, tokens, vocab, _lib.ptr(proposals),
                _lib.ptr(first), None, _lib.ptr(pred), _lib.ptr(acc), _lib.ptr(nxt), stream)
            torch.cuda.synchronize()
            outs[entry] = (status, pred.cpu().numpy(), acc.cpu().numpy(), nxt.cpu().numpy())
        status, *got = outs["carat_hip_argmax_accept_noalloc"]
        want = outs["carat_hip_argmax_accept"]
        assert want[0] == 0
        if requests == 256:
            assert status == 0
            for a, b in zip(got, want[1:]):
                assert np.array_equal(a, b)
        else:
            assert status != 0
            assert "exceed the fixed scratch of 65536" in _lib.lib().carat_hip_last_error().decode()
            assert all(np.all(a == -7) for a in got)
        del logits
