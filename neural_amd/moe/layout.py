"""Expert geometry of the GPT-OSS-120B MXFP4 store: byte layout of one expert slot and the u8 views over a slot pool.

Mirrors the public surface of the reference's ``neural/moe/layout.py`` (``MXFP4_REPRS``, ``packed_scale_row_bytes``,
``ExpertLayout``, ``GPTOSS_LAYOUT``, ``GPTOSS_LAYOUT_PS4``, ``gptoss_layout_for_repr``, ``mxfp4_pool_views``,
``prepacked_descriptor``; reference layout.py:17-212) for the two MXFP4 representations only.  The int4/int6/int8
Qwen representations of the reference are outside this path and are refused.

Slot byte order (reference layout.py:103-106, tools/scale_pack.py:6-12):

    gate_codes [gate_up_n][GK][16] | down_codes [down_n][GK][16] | gate_scales | down_scales

with GK = K/32 groups per row, 16 code bytes per group (two E2M1 codes per byte, low nibble = even element) and the
scale region either one E8M0 byte per group (``mxfp4_g32``) or, per row, one base byte followed by GK/2 bytes of
4-bit deltas (``mxfp4_g32_ps4``; low nibble = even group).

A third representation, ``mxfp4_g32_t950``, is this build's gfx950 tile layout (neural_amd.tiles): the same logical
codes and scales, permuted so that one wavefront-wide 128-bit load is one dense tile.  It has no counterpart in the
reference; it round-trips bit-exactly to the raw slot.
"""
from __future__ import annotations

from dataclasses import dataclass

MXFP4_REPRS = ("mxfp4_g32", "mxfp4_g32_ps4")
TILE_REPR = "mxfp4_g32_t950"
_KNOWN_REPRS = MXFP4_REPRS + (TILE_REPR,)


def packed_scale_row_bytes(n_groups: int) -> int:
    """Bytes of one PS4 scale row: the base byte plus one nibble per group (reference layout.py:20-23)."""
    assert n_groups % 2 == 0
    return 1 + n_groups // 2


@dataclass(frozen=True)
class ExpertLayout:
    """Geometry of one MoE layer's experts; field names and meanings follow reference layout.py:26-52."""
    name: str
    n_layers: int
    n_experts: int
    top_k: int
    hidden: int          # K of the gate_up product
    gate_up_n: int       # N of the gate_up product (= 2 * intermediate, [gate | up] rows)
    down_n: int          # N of the down product (= hidden)
    down_k: int          # K of the down product (= intermediate)
    int4_group: int = 32
    inner_k_tiles: int = 2
    act: str = "swiglu"
    act_alpha: float = 1.0
    act_limit: float = 0.0
    has_expert_bias: bool = False
    weight_repr: str = "mxfp4_g32"

    def __post_init__(self):
        if self.weight_repr not in _KNOWN_REPRS:
            raise ValueError(f"weight_repr {self.weight_repr!r}: this build serves {_KNOWN_REPRS}")
        assert self.hidden % self.int4_group == 0 and self.down_k % self.int4_group == 0
        assert self.gate_up_n == 2 * self.down_k, "gate_up stacks gate|up over the intermediate"
        if self.weight_repr == "mxfp4_g32_ps4":
            assert (self.hidden // self.int4_group) % 2 == 0 and (self.down_k // self.int4_group) % 2 == 0, \
                "mxfp4_g32_ps4 needs an even number of scale groups per row"

    # ---- byte counts (reference layout.py:65-106, mxfp4 branches)
    @property
    def gate_pack_bytes(self) -> int:
        return self.gate_up_n * self.hidden // 2

    @property
    def down_pack_bytes(self) -> int:
        return self.down_n * self.down_k // 2

    def _scale_row(self, k: int) -> int:
        g = k // self.int4_group
        return packed_scale_row_bytes(g) if self.weight_repr == "mxfp4_g32_ps4" else g

    @property
    def gate_saz_bytes(self) -> int:
        return self._scale_row(self.hidden) * self.gate_up_n

    @property
    def down_saz_bytes(self) -> int:
        return self._scale_row(self.down_k) * self.down_n

    @property
    def slot_bytes(self) -> int:
        if self.weight_repr == TILE_REPR:
            # 16-row blocks of 24,576 B: codes in MFMA-operand tiles, then 16 padded 96-byte E8M0 rows
            return (self.gate_up_n + self.down_n) // 16 * (self.hidden // 2 * 16 + 16 * 96)
        return self.gate_pack_bytes + self.down_pack_bytes + self.gate_saz_bytes + self.down_saz_bytes

    @property
    def is_mxfp4(self) -> bool:
        return self.weight_repr in MXFP4_REPRS

    @property
    def scale_layout_mode(self) -> int:
        """0 = raw E8M0 byte per group, 1 = PS4 (base + 4-bit deltas); the CPU kernels' gptoss_set_scale_layout code."""
        return 1 if self.weight_repr == "mxfp4_g32_ps4" else 0

    # ---- derived offsets used by the native launchers
    @property
    def gate_groups(self) -> int:
        return self.hidden // self.int4_group

    @property
    def down_groups(self) -> int:
        return self.down_k // self.int4_group

    @property
    def off_down_codes(self) -> int:
        return self.gate_pack_bytes

    @property
    def off_gate_scales(self) -> int:
        return self.gate_pack_bytes + self.down_pack_bytes

    @property
    def off_down_scales(self) -> int:
        return self.off_gate_scales + self.gate_saz_bytes

    def descriptor(self) -> dict:
        return {"layout_name": self.name, "n_layers": self.n_layers,
                "n_experts": self.n_experts, "top_k": self.top_k,
                "hidden": self.hidden, "gate_up_n": self.gate_up_n,
                "down_n": self.down_n, "down_k": self.down_k,
                "int4_group": self.int4_group, "inner_k_tiles": self.inner_k_tiles,
                "slot_bytes": self.slot_bytes}


_GPTOSS = dict(n_layers=36, n_experts=128, top_k=4, hidden=2880, gate_up_n=5760, down_n=2880, down_k=2880,
               act="clamped_swiglu", act_alpha=1.702, act_limit=7.0, has_expert_bias=True)

GPTOSS_LAYOUT = ExpertLayout("gpt-oss-120b", weight_repr="mxfp4_g32", **_GPTOSS)
GPTOSS_LAYOUT_PS4 = ExpertLayout("gpt-oss-120b-ps4", weight_repr="mxfp4_g32_ps4", **_GPTOSS)
GPTOSS_LAYOUT_T950 = ExpertLayout("gpt-oss-120b-t950", weight_repr=TILE_REPR, **_GPTOSS)
assert GPTOSS_LAYOUT_T950.slot_bytes == 13_271_040
# raw slot byte count: codes 8,294,400 + 4,147,200, scales 518,400 + 259,200 (reference layout.py:147,155)
assert GPTOSS_LAYOUT.slot_bytes == 13_219_200
assert GPTOSS_LAYOUT_PS4.slot_bytes == 12_839_040
assert GPTOSS_LAYOUT_PS4.gate_pack_bytes == GPTOSS_LAYOUT.gate_pack_bytes
assert GPTOSS_LAYOUT_PS4.down_pack_bytes == GPTOSS_LAYOUT.down_pack_bytes
assert (GPTOSS_LAYOUT.scale_layout_mode, GPTOSS_LAYOUT_PS4.scale_layout_mode) == (0, 1)

_GPTOSS_STORE_LAYOUTS = {"mxfp4_g32": GPTOSS_LAYOUT, "mxfp4_g32_ps4": GPTOSS_LAYOUT_PS4}


def gptoss_layout_for_repr(weight_repr: str) -> ExpertLayout:
    """The gpt-oss layout a store descriptor's ``weight_repr`` names (KeyError for anything else)."""
    return _GPTOSS_STORE_LAYOUTS[weight_repr]


def mxfp4_pool_views(pool, L: ExpertLayout):
    """(gate_blocks, down_blocks, gate_scales, down_scales) u8 views over a slot pool ``pool`` [cap, L.slot_bytes]:
    blocks [cap, N, GK, 16]; scales [cap, N, GK] raw or [cap, N, GK//2 + 1] PS4.  Slot-strided views
    (stride(0) == slot_bytes), exactly the shapes the reference's kernels consume (reference layout.py:168-186)."""
    assert L.is_mxfp4, L.weight_repr
    assert pool.dim() == 2 and pool.shape[1] == L.slot_bytes, (tuple(pool.shape), L.slot_bytes)
    cap = pool.shape[0]
    g_end = L.gate_pack_bytes
    d_end = g_end + L.down_pack_bytes
    gs_end = d_end + L.gate_saz_bytes
    gg, dg = L.gate_groups, L.down_groups
    gw, dw = L._scale_row(L.hidden), L._scale_row(L.down_k)
    return (pool[:, :g_end].view(cap, L.gate_up_n, gg, 16),
            pool[:, g_end:d_end].view(cap, L.down_n, dg, 16),
            pool[:, d_end:gs_end].view(cap, L.gate_up_n, gw),
            pool[:, gs_end:].view(cap, L.down_n, dw))


def prepacked_descriptor(layout: ExpertLayout) -> dict:
    """The identity descriptor a store's metadata.json carries for ``layout`` (keys and values of reference
    layout.py:189-212 for the mxfp4 representations, so existing stores stay byte-compatible)."""
    d = {"slot_bytes": layout.slot_bytes, "n_layers": layout.n_layers,
         "n_experts": layout.n_experts, "hidden": layout.hidden,
         "gate_up_n": layout.gate_up_n, "down_n": layout.down_n,
         "down_k": layout.down_k, "int4_group": layout.int4_group,
         "inner_k_tiles": layout.inner_k_tiles,
         "weight_repr": layout.weight_repr}
    if layout.weight_repr == "mxfp4_g32":
        d["row"] = "gate_codes|down_codes|gate_scales|down_scales"
        d["kernel"] = "neural.q80.mxfp4_kernels (Triton, fp32-accum)"
    elif layout.weight_repr == "mxfp4_g32_ps4":
        d["row"] = "gate_codes|down_codes|gate_scales_ps4|down_scales_ps4"
        d["kernel"] = "neural.q80.mxfp4_kernels (Triton, fp32-accum, packed 4-bit scale deltas)"
    else:
        d["row"] = "gfx950 tiles: gate_tiles|down_tiles (codes and E8M0 scales interleaved per tile)"
        d["kernel"] = "neural_amd (HIP gfx950, fp32-accum)"
    return d
