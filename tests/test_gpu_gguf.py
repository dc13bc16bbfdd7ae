"""Real GGUF bytes feeding the kernels: kq_gguf_open's descriptors passed
to kq_linear_init / kq_linear_dispatch unchanged, the type-42 file from
kq_gguf_nib_convert, and the device-side Q2_K -> type-42 permutation
(kq_q2k_to_nib_dev) against the oracle's permutation (pinned against the
reference converter by tests/test_oracle.py and tests/test_gguf.py).

Bars: permutation bit-exact; GEMVs through the index at the GEMV contract
(1e-5 relative, argmax identical, bit-identical count printed); a type-42
tensor gives the same outputs as its Q2_K source, bit for bit.
"""
import numpy as np
import pytest

import gguf_build as G
import stratum_amd as K
from conftest import same_values
from oracle import oracle as O
from stratum_amd import gguf as KG
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


@pytest.mark.parametrize("nblocks", [1, 37, 4096, 100003])
def test_q2k_to_nib_dev_bit_exact(port, nblocks):
    q2k = synth.q2k_blocks(synth.rng(9700 + nblocks), nblocks)
    src = torch.from_numpy(q2k).cuda()
    dst = torch.full((nblocks * 148,), 0x5A, dtype=torch.uint8, device="cuda")
    print(f"q2k_to_nib nblocks={nblocks}", flush=True)
    KG.q2k_to_nib_dev(src.data_ptr(), dst.data_ptr(), nblocks,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), port.q2k_to_nib(q2k))


def test_model_file_through_the_index(port):
    r = synth.rng(9800)
    H = 1024
    specs = [("blk.0.attn_q.weight", 12, 512), ("blk.0.ffn_down.weight", 14, 300),
             ("blk.0.ffn_gate.weight", 10, 256), ("blk.0.ffn_up.weight", 13, 200),
             ("blk.0.attn_v.weight", 8, 128), ("blk.0.attn_k.weight", 0, 64)]
    ts = [(name, [H, N], t, synth.tensor(t, N, H, 9801 + i).tobytes())
          for i, (name, t, N) in enumerate(specs)]
    buf = G.model(ts, [G.kv_str("general.architecture", "llama")], align=32)
    ix = KG.Index(buf)
    K.WeightRegion(buf)
    x = synth.gaussian(synth.rng(9899), H)
    for name, t, N in specs:
        d = ix.find(name)
        assert d is not None and d.type == t
        w = buf[d.offset:d.offset + d.nbytes]
        got = K.linear_dispatch(d, x, N, H)
        want = port.gemv(t, w, x, N, H)
        rel = O.rel_err(got, want).max()
        print(f"{name} type {t}: max rel {rel:.2e}, bit-identical "
              f"{int(np.sum(got == want))}/{N}", flush=True)
        assert rel <= 1e-5 and np.argmax(got) == np.argmax(want), name
    # the same model converted to type 42: the Q2_K tensor keeps its outputs
    conv, n = ix.nib_convert()
    assert n == 1
    iy = KG.Index(conv)
    K.WeightRegion(conv)
    d0 = ix.find("blk.0.ffn_gate.weight")
    d1 = iy.find("blk.0.ffn_gate.weight")
    assert d1.type == 42
    y42 = K.linear_dispatch(d1, x, 256, H)
    K.WeightRegion(buf)
    assert same_values(y42, K.linear_dispatch(d0, x, 256, H))
    for name, t, N in specs:        # the other tensors moved but did not change
        if t != 10:
            K.WeightRegion(conv)
            a = K.linear_dispatch(iy.find(name), x, N, H)
            K.WeightRegion(buf)
            assert same_values(a, K.linear_dispatch(ix.find(name), x, N, H)), name
