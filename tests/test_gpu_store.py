"""Loading a prepacked store into HBM (neural_amd.moe.gptoss_adapter.load_resident_store) on the GPU.

A raw and a PS4 store of the same 8 synthetic slots (2 layers x 4 experts) with biases: loaded with the tile repack
(in chunks of 3 slots, so partial chunks and both staging buffers are exercised) both give the pool that
repack_to_t950 makes from the slots directly, bit for bit; loaded without it the pool rows are the store rows; the
loaded runtime's decode output (biases included) matches the oracle's expert forward within the expert tolerance.
"""
import dataclasses

import numpy as np
import pytest

from oracle import mxfp4_oracle as mo
from oracle.bf16 import rb

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stores(tmp_path_factory):
    import torch
    from neural_amd import scale_pack as sp
    from neural_amd import synth
    from neural_amd.moe.gptoss_adapter import GPTOSS_MODEL_ID
    from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4
    from neural_amd.q80.prepacked_store import Q80PrepackedStore

    rng = np.random.default_rng(17)
    slots = [synth.slot_raw(rng) for _ in range(8)]
    raw = dataclasses.replace(GPTOSS_LAYOUT, n_layers=2, n_experts=4)
    pk = dataclasses.replace(GPTOSS_LAYOUT_PS4, n_layers=2, n_experts=4)
    g = torch.Generator().manual_seed(5)
    biases = ((torch.randn(8, 5760, generator=g) * 0.05).to(torch.bfloat16),
              (torch.randn(8, 2880, generator=g) * 0.05).to(torch.bfloat16))
    base = tmp_path_factory.mktemp("gstores")
    src, dst = str(base / "raw"), str(base / "ps4")
    Q80PrepackedStore.build(src, lambda li, e: slots[4 * li + e], model_id=GPTOSS_MODEL_ID, layout=raw, biases=biases)
    Q80PrepackedStore.build(dst, lambda li, e: sp.pack_slot(slots[4 * li + e]), model_id=GPTOSS_MODEL_ID, layout=pk,
                            biases=biases)
    return dict(slots=slots, raw=raw, pk=pk, src=src, dst=dst, biases=biases)


def test_load_with_tile_repack_equals_direct_repack(stores):
    import torch
    from neural_amd import tiles
    from neural_amd.moe.gptoss_adapter import load_resident_store

    dev = torch.device("cuda", 0)
    print("case store load raw + ps4 -> t950", flush=True)
    a = load_resident_store(stores["src"], dev, layout=stores["raw"], chunk=3, verify=True)
    b = load_resident_store(stores["dst"], dev, layout=stores["pk"], chunk=3)
    src = torch.from_numpy(np.stack(stores["slots"])).to(dev)
    want = torch.empty_like(a["pool"])
    tiles.repack_to_t950(src, want)
    torch.cuda.synchronize()
    assert torch.equal(a["pool"], want) and torch.equal(b["pool"], want)
    assert torch.equal(a["bias_gu"].cpu(), stores["biases"][0]) and torch.equal(b["bias_dn"].cpu(), stores["biases"][1])
    assert a["layout"].weight_repr == "mxfp4_g32_t950" and a["layout"].n_experts == 4
    print(f"loaded {a['pool'].shape[0]} slots at {a['gbps']:.2f} GB/s", flush=True)


def test_load_without_repack_keeps_store_rows(stores):
    import torch
    from neural_amd.moe.gptoss_adapter import load_resident_store

    dev = torch.device("cuda", 0)
    print("case store load raw, no repack", flush=True)
    a = load_resident_store(stores["src"], dev, layout=stores["raw"], tiles=False, chunk=3)
    torch.cuda.synchronize()
    assert np.array_equal(a["pool"].cpu().numpy(), np.stack(stores["slots"]))


def test_loaded_runtime_decode_matches_oracle(stores):
    import torch
    from neural_amd.moe.gptoss_adapter import load_resident_store

    dev = torch.device("cuda", 0)
    print("case store load -> decode layer 1", flush=True)
    a = load_resident_store(stores["dst"], dev, layout=stores["pk"], chunk=4, max_batch=1)
    rx = a["runtime"]
    rng = np.random.default_rng(4)
    x = rb(rng.standard_normal((1, 2880)).astype(np.float32))
    ids = np.array([[2, 0, 3, 1]], np.int64)
    w = rb(np.array([[0.4, 0.3, 0.2, 0.1]], np.float32))
    out = rx.forward_decode(1, torch.from_numpy(x).to(torch.bfloat16).to(dev), torch.from_numpy(ids).to(dev),
                            torch.from_numpy(w).to(torch.bfloat16).to(dev))
    torch.cuda.synchronize()
    bgu, bdn = (t.float().numpy() for t in stores["biases"])
    ys = [mo.expert_forward_bf16(x, stores["slots"][4 + e], bgu[4 + e], bdn[4 + e])[0] for e in ids[0]]
    want = mo.combine_bf16(np.stack(ys), w[0])
    got = out.float().cpu().numpy()[0]
    assert np.abs(got - want).max() <= 2e-2 + 1e-2 * np.abs(want).max()
