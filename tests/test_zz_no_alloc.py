"""fs_spec_accept_noalloc (the acceptance with its scratch in the library's fixed device array)
against fs_spec_accept (the same kernels on a caller workspace): identical tokens, counts and
rollback lengths, on two calls in a row, the second with a smaller batch, vocabulary and k, with and
without the rows' statistics given, and replayed from a HIP graph; a shape whose scratch exceeds the
array is refused before any launch."""

import pytest
import torch

from forgeserve_amd import _lib, ops
from forgeserve_amd._lib import DTYPE_CODE, ptr, stream_ptr
from oracle import reference_cpu as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(*a):
    print("case:", *a, flush=True)


def _inputs(b, k, v, seed):
    g = torch.Generator().manual_seed(seed)
    tgt = (torch.randn(b, k + 1, v, generator=g) * 2).bfloat16()
    dft = (tgt[:, :k].float() + torch.randn(b, k, v, generator=g) * 0.5).bfloat16()
    temps = torch.tensor([(0.0, 0.7, 1.0, 1.3)[i % 4] for i in range(b)])
    xs = torch.zeros(b, k, dtype=torch.int32)
    for bi in range(b):
        for i in range(k):
            t = float(temps[bi])
            xs[bi, i] = int(dft[bi, i].float().argmax()) if t == 0 else \
                orc.draw(orc.probs_from_logits(dft[bi, i], t), orc.exp_noise(v, g))
    u = torch.rand(b, k, generator=g)
    e = torch.empty(b, v).exponential_(generator=g)
    k_eff = torch.tensor([k - (i % (k + 1)) for i in range(b)], dtype=torch.int32)
    seq = torch.randint(10, 1000, (b,), generator=g, dtype=torch.int32)
    return [x.to(DEV) for x in (tgt, dft, xs, k_eff, temps, u, e, seq)]


def _records(tgt, dft, temps):
    """Merged softmax statistics of the 2k+1 rows (as the LM head's epilogue would give them)."""
    rows = torch.cat([tgt, dft], 1).float()
    t = temps[:, None, None]
    y = torch.where(t > 0, rows / t.clamp(min=1e-30), rows)
    mx = y.max(-1).values
    f = torch.stack([mx, torch.exp((y - mx[..., None]).double()).sum(-1).float(), rows.max(-1).values], -1)
    return torch.cat([f.contiguous().view(torch.int32), rows.argmax(-1).to(torch.int32)[..., None]], -1).contiguous()


def _noalloc(tgt, dft, xs, k_eff, temps, u, e, seq, row_stats, out=None, n=None):
    b, k1, v = tgt.shape
    k = k1 - 1
    if out is None:
        out = torch.full((b, k + 1), -7, dtype=torch.int32, device=DEV)
        n = torch.full((b,), -7, dtype=torch.int32, device=DEV)
    rc = _lib.load().fs_spec_accept_noalloc(ptr(tgt), tgt.stride(0), tgt.stride(1), ptr(dft), dft.stride(0),
                                            dft.stride(1), b, k, v, DTYPE_CODE[tgt.dtype], ptr(xs), ptr(k_eff),
                                            ptr(temps), ptr(u), ptr(e), e.stride(0), ptr(row_stats), ptr(out), ptr(n),
                                            ptr(seq), stream_ptr())
    _lib.check(rc, "spec_accept_noalloc")
    return out, n


@pytest.mark.parametrize("with_stats", [False, True])
def test_noalloc_acceptance_equals_the_workspace_entry_point(with_stats):
    for b, k, v in ((64, 6, 128256), (9, 3, 32000)):   # the second call is smaller in every dimension
        case("spec_accept_noalloc", b, k, v, "row statistics" if with_stats else "statistics pass")
        tgt, dft, xs, k_eff, temps, u, e, seq = _inputs(b, k, v, b + k)
        st = _records(tgt, dft, temps) if with_stats else None
        seq_ref = seq.clone()
        want_out, want_n = ops.spec_accept(tgt, dft, xs, k_eff, temps, u, e, seq_len=seq_ref, row_stats=st)
        got_out, got_n = _noalloc(tgt, dft, xs, k_eff, temps, u, e, seq, st)
        torch.cuda.synchronize()
        assert torch.equal(got_out, want_out) and torch.equal(got_n, want_n)
        assert torch.equal(seq, seq_ref)
        assert int(want_n.sum()) > 0   # some proposals were accepted, so the accepted prefixes were compared


@pytest.mark.parametrize("with_stats", [False, True])
def test_noalloc_acceptance_under_graph_capture(with_stats):
    """After an eager call (the first call on a device looks the scratch up and clears it, which must not
    be captured), a call captured into a HIP graph and replayed three times, with eager work and
    synchronisations between the replays, gives fs_spec_accept's outputs on every replay."""
    case("spec_accept_noalloc graph", "row statistics" if with_stats else "statistics pass")
    b, k, v = 16, 4, 32000
    tgt, dft, xs, k_eff, temps, u, e, seq = _inputs(b, k, v, 5)
    st = _records(tgt, dft, temps) if with_stats else None
    seq0 = seq.clone()
    seq_ref = seq0.clone()
    want_out, want_n = ops.spec_accept(tgt, dft, xs, k_eff, temps, u, e, seq_len=seq_ref, row_stats=st)
    out = torch.full((b, k + 1), -7, dtype=torch.int32, device=DEV)
    n = torch.full((b,), -7, dtype=torch.int32, device=DEV)
    _noalloc(tgt, dft, xs, k_eff, temps, u, e, seq, st, out, n)   # eager: the device's first call, if it is
    torch.cuda.synchronize()
    assert torch.equal(out, want_out) and torch.equal(n, want_n) and torch.equal(seq, seq_ref)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            _noalloc(tgt, dft, xs, k_eff, temps, u, e, seq, st, out, n)
    torch.cuda.current_stream().wait_stream(side)
    x = torch.randn(512, 512, device=DEV)
    for rep in range(3):
        seq.copy_(seq0)
        out.fill_(-7)
        n.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        y = x @ x   # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, want_out) and torch.equal(n, want_n), rep
        assert torch.equal(seq, seq_ref), rep
        assert float(y.abs().sum()) > 0


def test_noalloc_refuses_shapes_beyond_its_scratch():
    case("spec_accept_noalloc refusal")
    lib = _lib.load()
    dummy = torch.zeros(16, dtype=torch.int32, device=DEV)
    p = ptr(dummy)
    # batch 4096 at k = 8 and V = 128256 needs ~28 MiB of scratch: refused on the host, nothing launched
    rc = lib.fs_spec_accept_noalloc(p, 0, 0, p, 0, 0, 4096, 8, 128256, 1, p, p, p, p, p, 128256, None, p, p, None,
                                    stream_ptr())
    assert rc == -1 and b"scratch" in lib.fs_last_error()
