"""The MoE block's down-projection surface (hsd/model.py:53-175, MoEBlock) and the
one-layer-at-a-time layout build of NemotronModel.set_mode (hsd/model.py:233-252).

MoEDown holds one MoE layer's down projections: the checkpoint's stock layout (routed
`fc2` w [E, D, F/8] u32, s/b [E, D, F/64] bf16; shared `down_proj` w [D, FS/8], s/b
[D, FS/64]) and, after build_layout, the neuron-major layout the sparse kernels read.
With drop_stock the stock tensors are released, so one layout per layer stays resident
(hsd AGENTS.md:47-49).

The front end (norm, router, up projections, ReLU^2; model.py:110-121) is not on this
path: its outputs (inds, scores, h, hs) are arguments of pack / decode_sparse /
prefill_sparse, which then do what model.py:123-139 and 156-175 do after the front end:
pack, the sparse down projection, and the residual add.
"""
import torch

from . import _native as N
from . import decode, layout, prefill


class MoEDown:
    """hsd/model.py MoEBlock, its down-projection half. fc2 and shared_down are dicts with
    "weight", "scales" and "biases" (device tensors, the checkpoint's stock layout).
    decode_kw / prefill_kw are passed to sparse_down / sparse_down_prefill (the Metal
    knobs there are accepted and ignored; prefill_kw["tt"] selects 32- or 64-slot
    tiles)."""

    def __init__(self, fc2, shared_down, *, topk, decode_kw=None, prefill_kw=None):
        w, sw = fc2["weight"], shared_down["weight"]
        if w.dim() != 3 or sw.dim() != 2:
            raise N.HSDError("fc2 weight must be [E, D, F/8] and the shared weight [D, FS/8]")
        self.E, self.D, self.F = w.shape[0], w.shape[1], w.shape[2] * 8
        self.FS = sw.shape[1] * 8
        if sw.shape[0] != self.D:
            raise N.HSDError("routed and shared down projections disagree on D")
        self.topk = topk
        self.fc2 = {k: fc2[k] for k in ("weight", "scales", "biases")}
        self.shared_down = {k: shared_down[k] for k in ("weight", "scales", "biases")}
        self.decode_kw = dict(decode_kw or {})
        self.prefill_kw = dict(tt=32)
        self.prefill_kw.update(prefill_kw or {})
        self.pw = self.ps = self.pb = self.spw = self.sps = self.spb = None
        self.has_layout = False
        self.stock_layout = True

    @property
    def w_routed(self):
        """(pw, ps, pb): the routed experts' down projection, neuron-major."""
        return (self.pw, self.ps, self.pb)

    @property
    def w_shared(self):
        """(spw, sps, spb): the shared expert's down projection, neuron-major."""
        return (self.spw, self.sps, self.spb)

    def build_layout(self, drop_stock=True):
        """model.py:89-100. The neuron-major layout (an exact permutation of the stock bytes,
        hsd.layout), then, with drop_stock, the stock tensors released."""
        if not self.stock_layout:
            raise N.HSDError("the stock layout was dropped; the neuron-major one cannot be rebuilt")
        f, s = self.fc2, self.shared_down
        self.pw, self.ps, self.pb = layout.to_neuron_major(f["weight"], f["scales"], f["biases"])
        self.spw, self.sps, self.spb = layout.to_neuron_major(s["weight"], s["scales"], s["biases"])
        self.has_layout = True
        if drop_stock:
            self.drop_stock()

    def drop_stock(self):
        """model.py:102-107: the stock down projections are freed (the references to them
        dropped; the caching allocator reuses the bytes for the next layer)."""
        self.fc2 = None
        self.shared_down = None
        self.stock_layout = False

    def pack(self, inds, scores, h, hs):
        """model.py:123-129. h [B, topk, (1,) F] and hs [B, FS] after ReLU^2 -> hcat
        [B, topk*F + FS] (the routed slots, then the shared expert, contiguous), sel
        [B, topk] int32, gains [B, topk + 1] f32 (the routing scores, then 1 for shared)."""
        B = h.shape[0]
        if h.numel() != B * self.topk * self.F or hs.shape != (B, self.FS):
            raise N.HSDError(f"pack: h must hold [B, {self.topk}, {self.F}] and hs [B, {self.FS}]")
        hcat = torch.cat([h.reshape(B, self.topk * self.F), hs.to(h.dtype)], dim=1).contiguous()
        ones = torch.ones((B, 1), dtype=torch.float32, device=scores.device)
        gains = torch.cat([scores.to(torch.float32), ones], dim=1).contiguous()
        return hcat, inds.to(torch.int32).contiguous(), gains

    def _need_layout(self):
        if not self.has_layout:
            raise N.HSDError("sparse mode needs the neuron-major layout (build_layout)")

    def decode_sparse(self, x, inds, scores, h, hs):
        """model.py:135-139 after the front end: x [B, D] + the sparse down projection."""
        self._need_layout()
        hcat, sel, gains = self.pack(inds, scores, h, hs)
        y = decode.sparse_down(hcat, sel, gains, *self.w_routed, *self.w_shared, F=self.F, FS=self.FS,
                               D=self.D, topk=self.topk, **self.decode_kw)
        return x + y.to(x.dtype)

    def decode_dense(self, x, inds, scores, h, hs):
        """The dense comparator on the stock layout (what dense mode's quantised matmuls
        compute, model.py:132-133): x [B, D] + the down projection over every row."""
        if not self.stock_layout:
            raise N.HSDError("dense mode needs the checkpoint's down layout, freed by build_layout")
        hcat, sel, gains = self.pack(inds, scores, h, hs)
        f, s = self.fc2, self.shared_down
        y = decode.dense_down(hcat, sel, gains, f["weight"], f["scales"], f["biases"], s["weight"],
                              s["scales"], s["biases"], F=self.F, FS=self.FS, D=self.D, topk=self.topk,
                              out_dtype=self.decode_kw.get("out_dtype"))
        return x + y.to(x.dtype)

    def prefill_sparse(self, x, inds, scores, h, hs):
        """model.py:156-175 after the front end: tile order, union lists and the grouped
        GEMM on the device, then x [T, D] + y. h is [T, topk, F] in token order."""
        self._need_layout()
        hcat, sel, gains = self.pack(inds, scores, h, hs)
        tt = self.prefill_kw["tt"]
        tiles = prefill.build_tiles(sel, self.E, tt)
        union = prefill.build_union(hcat, tiles[0], tiles[1], F=self.F, FS=self.FS, topk=self.topk,
                                    E=self.E, tt=tt)
        kw = {k: v for k, v in self.prefill_kw.items() if k != "tt"}
        y = prefill.sparse_down_prefill(hcat, sel, gains, *self.w_routed, *self.w_shared, F=self.F,
                                        FS=self.FS, D=self.D, topk=self.topk, E=self.E, tt=tt,
                                        tiles=tiles, union=union, **kw)
        return x + y.to(x.dtype)


def up_relu2(x, inds, w1, s1, b1, sw1, ss1, sb1, *, topk, live_masks=None, status=None, out=None):
    """The front end after the router (model.py:110-121) in pack's layout: x [B, D] bf16
    (the normed token), inds [B, topk] -> hcat [B, topk*F + FS] bf16 = square(relu(x W^T))
    of each selected expert's up projection (w1 [E, F, D/8] u32, s1/b1 [E, F, D/64] bf16,
    the stock layout), then the shared expert's (sw1 [FS, D/8], ss1/sb1 [FS, D/64]).
    live_masks: optional int64 tensor of B*(topk*F + FS)/64 entries that receives the
    canonical live mask of every 64-group of hcat. status: optional int32 [1], ORed with 1
    for an expert id outside [0, E) (that slot is then 0)."""
    if x.dtype != torch.bfloat16:
        raise N.HSDError("up_relu2 takes bf16 activations")
    x = N.contig(x)
    B, D = x.shape
    E, F = w1.shape[0], w1.shape[1]
    FS = sw1.shape[0]
    NR = topk * F + FS
    hcat = out if out is not None else torch.empty((B, NR), dtype=torch.bfloat16, device=x.device)
    if live_masks is not None and (live_masks.dtype != torch.int64 or not live_masks.is_contiguous()
                                   or live_masks.numel() < B * (NR // 64)):
        raise N.HSDError("live_masks must be a contiguous int64 tensor of B*(topk*F + FS)/64 entries")
    inds = inds if inds.dtype == torch.int32 and inds.is_contiguous() else N.contig(inds.to(torch.int32))
    N.call("hsd_moe_up_relu2", N.ptr(x), N.dtype_tag(x.dtype), N.ptr(inds),
           N.ptr(N.as_words(N.contig(w1))), N.ptr(N.contig(s1)), N.ptr(N.contig(b1)),
           N.ptr(N.as_words(N.contig(sw1))), N.ptr(N.contig(ss1)), N.ptr(N.contig(sb1)), N.ptr(hcat),
           B, D, F, FS, topk, E, N.ptr(live_masks), N.ptr(status), N.stream(x.device))
    return hcat


def route_up_relu2(x, logits, e_bias, w1, s1, b1, sw1, ss1, sb1, *, topk, routed_scale=1.0, norm_topk=True,
                   live_masks=None, out=None, sel=None, gains=None):
    """The MoE front end WITH the router (model.py:110-121 from `mix.gate` on): from the
    gate's logits [B, E] bf16 (nn.linear of the normed token with the bf16 gate weight)
    the top-k experts (sigmoid scores plus the selection bias e_bias [E] f32, descending,
    equal choices by expert id), their gains (normalised and scaled), then hcat as
    up_relu2. -> (hcat [B, topk*F + FS] bf16, sel [B, topk] int32, gains [B, topk+1] f32)."""
    if x.dtype != torch.bfloat16 or logits.dtype != torch.bfloat16:
        raise N.HSDError("route_up_relu2 takes bf16 activations and logits")
    x = N.contig(x)
    logits = N.contig(logits)
    B, D = x.shape
    E, F = w1.shape[0], w1.shape[1]
    FS = sw1.shape[0]
    NR = topk * F + FS
    hcat = out if out is not None else torch.empty((B, NR), dtype=torch.bfloat16, device=x.device)
    sel = sel if sel is not None else torch.empty((B, topk), dtype=torch.int32, device=x.device)
    gains = gains if gains is not None else torch.empty((B, topk + 1), dtype=torch.float32, device=x.device)
    N.call("hsd_moe_route_up_relu2", N.ptr(x), N.DT_BF16, N.ptr(logits), N.ptr(e_bias), float(routed_scale),
           1 if norm_topk else 0, N.ptr(sel), N.ptr(gains), N.ptr(N.as_words(N.contig(w1))), N.ptr(N.contig(s1)),
           N.ptr(N.contig(b1)), N.ptr(N.as_words(N.contig(sw1))), N.ptr(N.contig(ss1)), N.ptr(N.contig(sb1)),
           N.ptr(hcat), B, D, F, FS, topk, E, N.ptr(live_masks), N.stream(x.device))
    return hcat, sel, gains


def router_topk(logits, e_bias, *, topk, routed_scale=1.0, norm_topk=True, sel=None, gains=None):
    """The router's selection from the gate's logits [B, E] bf16 (model.py:115): -> (sel
    [B, topk] int32, gains [B, topk+1] f32), by route_up_relu2's rule."""
    logits = N.contig(logits)
    B, E = logits.shape
    sel = sel if sel is not None else torch.empty((B, topk), dtype=torch.int32, device=logits.device)
    gains = gains if gains is not None else torch.empty((B, topk + 1), dtype=torch.float32, device=logits.device)
    N.call("hsd_router_topk", N.ptr(logits), N.ptr(e_bias), float(routed_scale), 1 if norm_topk else 0, N.ptr(sel),
           N.ptr(gains), B, E, topk, N.stream(logits.device))
    return sel, gains


def build_layouts(blocks, single_layout=True):
    """NemotronModel.set_mode("sparse") (model.py:233-247): every block's neuron-major
    layout, one layer at a time, so the permutation's transient stays one layer's size
    and, with single_layout, each layer's stock bytes are released before the next one
    is permuted."""
    for blk in blocks:
        if not blk.has_layout:
            blk.build_layout(drop_stock=single_layout)
    return blocks
