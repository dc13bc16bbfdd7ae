"""Device entries that use the library's scratch (the matrix-core and int8
multi-stream GEMVs, the int8 MoE batch) enqueued on two streams at once:
each stream has its own scratch, so calls that overlap in time give the
same bits as the same calls run alone."""
import numpy as np
import pytest

import stratum_amd as K
from stratum_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()
    yield
    torch.cuda.synchronize()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_scratch_entries_on_two_streams():
    """Rounds of matrix-core MULTISEQ, int8 MULTISEQ and int8 MoE batch calls
    with different inputs, alternating between two streams with no
    synchronisation between them: every output equals the call run alone on
    the default stream, and the second stream holds scratch of its own."""
    L = K.lib()
    N, Kd, B = 1024, 2048, 16
    w = dev(synth.tensor(12, N, Kd, 9700))
    r = synth.rng(9701)
    xs = [dev(np.stack([synth.gaussian(r, Kd) for _ in range(B)]).reshape(-1)) for _ in range(2)]
    # an int8 MoE batch: 16 experts of 256 x 512, 8 tokens, top-4
    E, F, H, k, T = 16, 256, 512, 4, 8
    ew = dev(synth.tensor(12, E * F, H, 9702))
    sl = F * L.kq_row_bytes(12, H)
    sels = [dev(np.stack([r.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
                .reshape(-1)) for _ in range(2)]
    mx = [dev(np.stack([synth.gaussian(r, H) for _ in range(T)]).reshape(-1)) for _ in range(2)]

    def calls(i, y_mf, y_i8, y_moe, st):
        K.gemv_multix_mfma_dev(12, w.data_ptr(), xs[i].data_ptr(), y_mf.data_ptr(), B, N, Kd,
                               stream=st)
        K.gemv_multix_dev(12 | K.INT8_ACT, w.data_ptr(), xs[i].data_ptr(), y_i8.data_ptr(), B, N,
                          Kd, stream=st)
        op = K.moe_op(12 | K.INT8_ACT, F, H, [ew.data_ptr()], sl, mx[i].data_ptr(), k,
                      [y_moe.data_ptr()])
        K.moe_gemv_dev(op, sels[i].data_ptr(), T, k, E, st)

    def outs():
        return (torch.full((B * N,), float("nan"), device="cuda"),
                torch.full((B * N,), float("nan"), device="cuda"),
                torch.full((T * k * F,), float("nan"), device="cuda"))

    alone = []
    for i in range(2):
        o = outs()
        calls(i, *o, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        alone.append([t.cpu().numpy().view(np.uint32) for t in o])
    held = L.kq_scratch_bytes()
    s = [torch.cuda.Stream(), torch.cuda.Stream()]
    print("two streams: mfma, int8 multix, int8 moe", flush=True)
    got = []
    for rnd in range(6):
        for i in range(2):
            with torch.cuda.stream(s[i]):      # the NaN fill is ordered before the calls
                o = outs()
            calls(i, *o, s[i].cuda_stream)
            got.append((i, o))
    torch.cuda.synchronize()
    for i, o in got:
        for name, t, want in zip(("mfma", "int8 multix", "int8 moe"), o, alone[i]):
            assert np.array_equal(t.cpu().numpy().view(np.uint32), want), (name, i)
    assert L.kq_scratch_bytes() > held


def test_more_streams_than_scratch_sets():
    """Eighteen streams in turn through the matrix-core MULTISEQ entry: the
    library keeps 16 scratch sets, so the seventeenth and eighteenth streams
    take the least recently used sets (freed first); every call still gives
    the default stream's bits, and the scratch held stays bounded."""
    L = K.lib()
    N, Kd, B = 256, 1024, 16
    w = dev(synth.tensor(12, N, Kd, 9710))
    r = synth.rng(9711)
    x = dev(np.stack([synth.gaussian(r, Kd) for _ in range(B)]).reshape(-1))
    want = torch.empty(B * N, device="cuda")
    K.gemv_multix_mfma_dev(12, w.data_ptr(), x.data_ptr(), want.data_ptr(), B, N, Kd,
                           stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = want.cpu().numpy().view(np.uint32)
    streams = [torch.cuda.Stream() for _ in range(18)]
    print("eighteen streams, matrix-core multix", flush=True)
    held = []
    for rnd in range(2):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                y = torch.full((B * N,), float("nan"), device="cuda")
            K.gemv_multix_mfma_dev(12, w.data_ptr(), x.data_ptr(), y.data_ptr(), B, N, Kd,
                                   stream=s.cuda_stream)
            s.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want), (rnd, i)
            held.append(L.kq_scratch_bytes())
    # after the first round the 16 sets are the last 16 streams' (whatever
    # earlier tests left): the second round only reassigns them, each one
    # freed and taken again at the same size
    assert all(h == held[17] for h in held[18:]), held
