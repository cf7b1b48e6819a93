"""The prepacked store reader/writer (neural_amd/q80/prepacked_store.py) and the gpt-oss adapter helpers
(neural_amd/moe/gptoss_adapter.py) on the CPU.

The contract is the reference's store behaviour (neural/q80/prepacked_store.py:149-230, gptoss_adapter.py:34-52):
layout_for_store names the layout from the descriptor alone and refuses missing, unreadable, foreign and
self-contradicting descriptors; a raw and a PS4 store of the same slots open with their own
layout and are refused with the other one (naming both representations); strict identity checks (magic, version,
model id, layer files); verify_layer catches a flipped byte; biases load through torch.load(weights_only=True).
The dequant helper is bit-exact against the oracle's dequant; the installer dispatches one token to decode and more
to prefill.
"""
import dataclasses
import json
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from neural_amd import scale_pack as sp
from neural_amd import synth
from neural_amd.moe import gptoss_adapter as GA
from neural_amd.moe.layout import GPTOSS_LAYOUT, GPTOSS_LAYOUT_PS4, GPTOSS_LAYOUT_T950
from neural_amd.q80.prepacked_store import Q80PrepackedStore
from oracle import mxfp4_oracle as mo

MID = GA.GPTOSS_MODEL_ID


def _metadata_only(root, layout, edit=None):
    """A store directory holding only metadata.json for ``layout`` (build() over no layers), optionally edited."""
    Q80PrepackedStore.build(root, None, model_id=MID, layout=layout, layers=())
    if edit is not None:
        p = os.path.join(root, "metadata.json")
        meta = json.load(open(p))
        edit(meta)
        json.dump(meta, open(p, "w"))
    return str(root)


def test_layout_for_store_reads_the_descriptor_only(tmp_path):
    raw = _metadata_only(tmp_path / "raw", GPTOSS_LAYOUT)
    ps4 = _metadata_only(tmp_path / "ps4", GPTOSS_LAYOUT_PS4)
    assert os.listdir(raw) == ["metadata.json"]          # no layer files: the layout comes from the metadata alone
    assert GA.layout_for_store(raw) is GPTOSS_LAYOUT and GA.layout_for_store(ps4) is GPTOSS_LAYOUT_PS4
    # a smaller store of the same representation still names the gpt-oss layout of that representation
    few = _metadata_only(tmp_path / "few", dataclasses.replace(GPTOSS_LAYOUT_PS4, n_layers=2))
    assert GA.layout_for_store(few) is GPTOSS_LAYOUT_PS4


def test_layout_for_store_refuses_what_it_cannot_name(tmp_path):
    os.makedirs(tmp_path / "empty")
    (tmp_path / "garbled").mkdir()
    (tmp_path / "garbled" / "metadata.json").write_text("{not json")
    cases = {
        "empty": str(tmp_path / "empty"),                                   # no metadata.json
        "garbled": str(tmp_path / "garbled"),                               # unreadable JSON
        "tiles": _metadata_only(tmp_path / "tiles", GPTOSS_LAYOUT_T950),    # this build's tile layout is no store
        "no_layout": _metadata_only(tmp_path / "nl", GPTOSS_LAYOUT, lambda m: m.update(layout="mxfp4_g32")),
        "no_repr": _metadata_only(tmp_path / "nr", GPTOSS_LAYOUT, lambda m: m["layout"].pop("weight_repr")),
        # raw slot size under the PS4 name, and the other way round: the descriptor contradicts itself
        "ps4_raw_size": _metadata_only(tmp_path / "c1", GPTOSS_LAYOUT_PS4,
                                       lambda m: m["layout"].update(slot_bytes=13_219_200)),
        "raw_ps4_size": _metadata_only(tmp_path / "c2", GPTOSS_LAYOUT,
                                       lambda m: m["layout"].update(slot_bytes=12_839_040)),
    }
    for name, root in cases.items():
        with pytest.raises(RuntimeError) as e:
            GA.layout_for_store(root)
        assert root in str(e.value), name
    with pytest.raises(RuntimeError, match="12839040 != 13219200"):
        GA.layout_for_store(cases["raw_ps4_size"])


@pytest.fixture(scope="module")
def stores(tmp_path_factory):
    """A raw and a PS4 store of the same two slots (one layer), with biases."""
    rng = np.random.default_rng(11)
    slots = [synth.slot_raw(rng) for _ in range(2)]
    raw = dataclasses.replace(GPTOSS_LAYOUT, n_layers=1, n_experts=2)
    pk = dataclasses.replace(GPTOSS_LAYOUT_PS4, n_layers=1, n_experts=2)
    g = torch.Generator().manual_seed(3)
    biases = ((torch.randn(2, 5760, generator=g) * 0.02).to(torch.bfloat16),
              (torch.randn(2, 2880, generator=g) * 0.02).to(torch.bfloat16))
    base = tmp_path_factory.mktemp("stores")
    src, dst = str(base / "raw"), str(base / "ps4")
    Q80PrepackedStore.build(src, lambda li, e: slots[e], model_id=MID, layout=raw, biases=biases)
    Q80PrepackedStore.build(dst, lambda li, e: sp.pack_slot(slots[e]), model_id=MID, layout=pk, biases=biases)
    return dict(slots=slots, raw=raw, pk=pk, src=src, dst=dst, biases=biases)


def test_store_files_and_metadata(stores):
    assert sorted(os.listdir(stores["dst"])) == ["expert_biases.pt", "layer_0.slots", "metadata.json"]
    meta = json.load(open(os.path.join(stores["dst"], "metadata.json")))
    assert meta["magic"] == "Q80-PREPACKED-SLOTS" and meta["version"] == 1 and meta["model_id"] == MID
    assert meta["layout"]["weight_repr"] == "mxfp4_g32_ps4" and meta["layout"]["slot_bytes"] == 12_839_040
    a = np.fromfile(os.path.join(stores["src"], "layer_0.slots"), np.uint8).reshape(2, sp.RAW_SLOT_BYTES)
    b = np.fromfile(os.path.join(stores["dst"], "layer_0.slots"), np.uint8).reshape(2, sp.PS4_SLOT_BYTES)
    for e in range(2):
        assert np.array_equal(a[e], stores["slots"][e])
        assert np.array_equal(sp.unpack_slot(b[e]), a[e])


def test_strict_open(stores):
    raw, pk = stores["raw"], stores["pk"]
    st = Q80PrepackedStore(stores["dst"], layout=pk)
    assert st.open(expect_model_id=MID)["status"] == "ok"
    assert (st.slot_bytes, st.weight_repr) == (12_839_040, "mxfp4_g32_ps4")
    assert np.array_equal(st.row(0, 1).numpy(), sp.pack_slot(stores["slots"][1]))
    buf = torch.empty(st.slot_bytes, dtype=torch.uint8)
    st.read_into(0, 0, buf)
    assert np.array_equal(buf.numpy(), sp.pack_slot(stores["slots"][0]))
    r = Q80PrepackedStore(stores["dst"], layout=raw).open(expect_model_id=MID)
    assert r["status"] == "fail" and r["store_weight_repr"] == "mxfp4_g32_ps4" and r["runtime_weight_repr"] == "mxfp4_g32"
    r = Q80PrepackedStore(stores["src"], layout=pk).open(expect_model_id=MID)
    assert r["status"] == "fail" and r["store_weight_repr"] == "mxfp4_g32"
    r = Q80PrepackedStore(stores["src"], layout=raw).open(expect_model_id="another-model")
    assert r == {"status": "fail", "reason": "model identity mismatch"}
    r = Q80PrepackedStore(stores["src"], layout=dataclasses.replace(raw, n_experts=3)).open()
    assert r["status"] == "fail" and r["differs"] == ["n_experts"]
    with pytest.raises(ValueError):
        Q80PrepackedStore(stores["src"])                               # the layout is required


def _copy_store(src, dst):
    os.makedirs(dst)
    for f in os.listdir(src):
        with open(os.path.join(src, f), "rb") as a, open(os.path.join(dst, f), "wb") as b:
            b.write(a.read())


def test_rejections_and_corruption(stores, tmp_path):
    raw = stores["raw"]
    d = str(tmp_path / "s")
    _copy_store(stores["src"], d)
    meta_p = os.path.join(d, "metadata.json")
    meta = json.load(open(meta_p))
    for key, val, reason in (("magic", "NOPE", "bad magic"), ("version", 2, "version 2 != 1")):
        m2 = dict(meta, **{key: val})
        json.dump(m2, open(meta_p, "w"))
        assert Q80PrepackedStore(d, raw).open() == {"status": "fail", "reason": reason}
    m2 = json.loads(json.dumps(meta))
    m2["layout"]["row"] = "a renamed label"                            # cosmetic: accepted with a note
    json.dump(m2, open(meta_p, "w"))
    r = Q80PrepackedStore(d, raw).open()
    assert r["status"] == "ok" and "row label differs" in r["descriptor_note"]
    json.dump(meta, open(meta_p, "w"))
    st = Q80PrepackedStore(d, raw)
    assert st.open()["status"] == "ok" and st.verify_layer(0)
    with open(os.path.join(d, "layer_0.slots"), "r+b") as f:            # one flipped byte
        f.seek(1234567)
        b = f.read(1)
        f.seek(1234567)
        f.write(bytes([b[0] ^ 0x10]))
    assert not st.verify_layer(0)
    with open(os.path.join(d, "layer_0.slots"), "ab") as f:            # wrong size
        f.write(b"\0")
    assert Q80PrepackedStore(d, raw).open() == {"status": "fail", "reason": "layer 0 missing/size"}
    os.remove(os.path.join(d, "layer_0.slots"))
    assert Q80PrepackedStore(d, raw).open() == {"status": "fail", "reason": "layer 0 missing/size"}
    os.remove(meta_p)
    assert Q80PrepackedStore(d, raw).open() == {"status": "fail", "reason": "no metadata.json"}


def test_biases_load_without_executing_anything(stores):
    st = Q80PrepackedStore(stores["src"], stores["raw"])
    assert st.open()["status"] == "ok"
    bgu, bdn = st.biases()
    assert torch.equal(bgu, stores["biases"][0]) and torch.equal(bdn, stores["biases"][1])


def test_fp4_table_dequant_and_deinterleave():
    assert np.array_equal(np.array(GA.FP4_VALUES), mo.E2M1)
    assert np.signbit(GA.FP4_VALUES[8]) and GA.FP4_VALUES[8] == 0.0
    rng = np.random.default_rng(2)
    slot = synth.slot_raw(rng)
    gc, dc, gs, ds = mo.slot_views(slot, False)
    want = mo.dequant_rows(gc[:64], gs[:64])
    got = GA.mxfp4_dequant_nk(torch.from_numpy(np.ascontiguousarray(gc[:64])),
                              torch.from_numpy(np.ascontiguousarray(gs[:64]))).numpy()
    assert np.array_equal(got, want.astype(np.float32))
    # the extreme scales: 255 (inf / nan for nonzero / zero codes in fp32) and 0 (2^-127, subnormal)
    blk = torch.tensor([[[0x21] * 16]], dtype=torch.uint8)
    out = GA.mxfp4_dequant_nk(blk, torch.tensor([[0]], dtype=torch.uint8))
    assert out[0, 0].item() == 0.5 * 2.0 ** -127 and out[0, 1].item() == 2.0 ** -127
    assert GA.deinterleave_perm(6).tolist() == [0, 2, 4, 1, 3, 5]


def test_installer_dispatch():
    calls = []
    rt = SimpleNamespace(forward_decode=lambda li, h, i, w: calls.append(("decode", li, h.shape[0])) or "d",
                         forward_prefill=lambda li, h, i, w: calls.append(("prefill", li, h.shape[0])) or "p")
    layers = [SimpleNamespace(mlp=SimpleNamespace(experts=SimpleNamespace(forward="orig"))) for _ in range(3)]
    model = SimpleNamespace(model=SimpleNamespace(layers=layers))
    inst = GA.install_gptoss_expert_runtime(rt, model)
    assert [o for _, o in inst] == ["orig"] * 3
    assert layers[1].mlp.experts.forward(torch.zeros(1, 4), None, None) == "d"
    assert layers[2].mlp.experts.forward(torch.zeros(5, 4), None, None) == "p"
    assert calls == [("decode", 1, 1), ("prefill", 2, 5)]
