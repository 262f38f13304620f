"""The Nemotron-H hybrid end to end on one MI355X (hsd/model.py: MoEBlock, NemotronModel).

A stack of Mamba-2 ("M"), MoE ("E") and GQA attention ("*") blocks, each `x + mixer(norm(x))`,
then norm_f and lm_head, plus the optional one-layer MTP head (hsd/mtp.py). Weights are
affine 4-bit group 64 (mlx's QuantizedLinear / QuantizedEmbedding format) except the router
gates and the MTP head's eh_proj (bf16). Every kernel is libhsd's:

  Mamba-2 block   nn.linear (rms_norm fused) -> hsd_mamba_ssm_gated (z and its 16-channel
                  sums of squares) -> nn.linear (gated norm + residual fused)   (mamba.py:19-44)
  MoE block       nn.linear of the bf16 gate (rms_norm fused, the normed token kept) ->
                  the router's top-k fused into the up projections + ReLU^2 -> the sparse
                  down projection with the residual fused        (model.py:110-139)
  attention block nn.linear q|k|v (rms_norm fused) -> nn.attention over the KV cache ->
                  nn.linear o_proj (residual fused)               (model.py:287, 343)
  lm_head         nn.linear with norm_f fused and the greedy argmax as its epilogue

The sequence state (cache lengths, Mamba ring index, emitted count, last token, ...) lives
in one device int32 array, so a decode step, a verify step with its acceptance and
rollback, and a whole MTP step each replay as one captured HIP graph with no host round
trip. Rows of a verify step are computed exactly as single decode rows, and the dense mode
runs the sparse kernel over every row (the dense-h control), so the three generation
modes produce bit-identical greedy tokens.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N
from . import layout, mamba as M, nn
from .moe import route_up_relu2, router_topk, up_relu2

NSLAB = 4          # Mamba checkpoint ring: a verify of up to 3 rows
ROWS = (1, 3)      # row counts with preallocated buffers: decode, verify / prefill steps


@dataclass
class ModelConfig:
    """The Nemotron-3.5-Lightning-30B-A3B shape (hybrid_override_pattern, 52 layers)."""
    hidden: int = 2688
    pattern: str = "MEMEM*EMEMEM*EMEMEM*EMEMEM*EMEMEM*EMEMEMEM*EMEMEMEME"
    vocab: int = 131072
    n_experts: int = 128
    topk: int = 6
    moe_inter: int = 1856
    shared_inter: int = 3712
    mamba_heads: int = 64
    mamba_head_dim: int = 64
    ssm_state: int = 128
    n_groups: int = 8
    attn_heads: int = 32
    kv_heads: int = 2
    head_dim: int = 128
    eps: float = 1e-5
    routed_scale: float = 2.5
    norm_topk: bool = True
    max_seq: int = 4096            # attention cache rows (prompt + generated + verify rows)
    mtp: bool = True               # the one-layer MTP head
    # synthetic-weight knobs (random init; see init_random)
    zero_frac: float = 0.9         # target ReLU^2 zero fraction of the MoE activations
    resid_scale: float = 0.25      # contribution scale of each block to the residual stream

    @property
    def mamba_inner(self):
        return self.mamba_heads * self.mamba_head_dim

    @property
    def conv_dim(self):
        return self.mamba_inner + 2 * self.n_groups * self.ssm_state

    @property
    def in_proj_dim(self):
        return 2 * self.mamba_inner + 2 * self.n_groups * self.ssm_state + self.mamba_heads

    @property
    def qkv_dim(self):
        return (self.attn_heads + 2 * self.kv_heads) * self.head_dim


# ------------------------------------------------------------------ random weights
class _Init:
    """Seeded synthetic weights drawn on the device. A 4-bit weight W = s q + b with
    uniform nibbles; s ~ U(0.75, 1.25) * std / 4.61 (4.61 = the std of a uniform nibble)
    and b = -7.5 s + N(0, 0.05 std), so W has mean ~0 and std ~std."""

    def __init__(self, seed, device):
        self.dev = device
        self.gen = torch.Generator(device=device)
        self.gen.manual_seed(seed)

    def q4(self, O, I, std, lead=()):
        g = self.gen
        w = torch.randint(-2 ** 31, 2 ** 31, (*lead, O, I // 8), dtype=torch.int32, device=self.dev, generator=g)
        s = (torch.rand((*lead, O, I // 64), device=self.dev, generator=g) * 0.5 + 0.75) * (std / 4.61)
        b = -7.5 * s + torch.randn((*lead, O, I // 64), device=self.dev, generator=g) * (0.05 * std)
        return w, s.to(torch.bfloat16), b.to(torch.bfloat16)

    def bf16(self, *shape, std=1.0):
        return (torch.randn(shape, device=self.dev, generator=self.gen) * std).to(torch.bfloat16)

    def uniform(self, *shape, lo=0.5, hi=1.5, dtype=torch.bfloat16):
        return (torch.rand(shape, device=self.dev, generator=self.gen) * (hi - lo) + lo).to(dtype)

    def normal_f32(self, *shape, std=1.0):
        return torch.randn(shape, device=self.dev, generator=self.gen) * std


def _zero_output_row0(w, s, b):
    """Output channel 0 of a stock-layout 4-bit projection is exactly 0 (q = s = b = 0):
    the blocks never write the residual stream's channel 0, which keeps the constant the
    embedding puts there (the synthetic model's bias channel)."""
    w[..., 0, :] = 0
    s[..., 0, :] = 0
    b[..., 0, :] = 0


# ------------------------------------------------------------------ blocks
class MambaBlock:
    """mlx-lm NemotronH "M" block: x + out_proj(gated_norm(ssm(conv(in_proj(norm(x))))))."""

    def __init__(self, cfg: ModelConfig, init: _Init):
        D = cfg.hidden
        self.norm_w = init.uniform(D)
        self.norm_w[0] = 0.0                               # the bias channel stays out of the mixer
        self.in_proj = nn.QWeight(*init.q4(cfg.in_proj_dim, D, 1.0 / math.sqrt(D)))
        w, s, b = init.q4(D, cfg.mamba_inner, cfg.resid_scale / math.sqrt(cfg.mamba_inner))
        _zero_output_row0(w, s, b)
        self.out_proj = nn.QWeight(w, s, b)
        H, CD = cfg.mamba_heads, cfg.conv_dim
        A_log = torch.log(init.uniform(H, lo=1.0, hi=16.0, dtype=torch.float32))
        Dp = init.uniform(H, lo=0.5, hi=1.5, dtype=torch.bfloat16).float()   # D as bf16 values
        self.mixer = M.Mamba2Mixer(conv_w=init.bf16(CD, 4, std=0.2), conv_b=init.bf16(CD, std=0.2), A_log=A_log,
                                   dt_bias=init.normal_f32(H, std=0.5), D=Dp, norm_w=init.uniform(cfg.mamba_inner),
                                   num_heads=H, head_dim=cfg.mamba_head_dim, ssm_state_size=cfg.ssm_state,
                                   n_groups=cfg.n_groups, norm_group=cfg.mamba_inner // cfg.n_groups, eps=cfg.eps)
        self.eps = cfg.eps

    def rows(self, x, buf, cache: M.MambaCache, status=None):
        """x [B, D] (updated in place). status: optional device int32 [1] (HSD_STATUS_*)."""
        B = x.shape[0]
        proj = nn.linear(x, self.in_proj, norm=self.norm_w, eps=self.eps, out=buf["proj"][:B])
        # the gate applied in the SSM kernel, which also leaves each 16 channels' sum of z^2
        # for out_proj's gated norm (no silu, no gate loads in its prologue)
        z = M.ssm_rows(self.mixer, proj, cache, out=buf["y_pre"][:B], gated=True, status=status)
        nn.linear(z, self.out_proj, norm=self.mixer.norm_w, eps=self.eps, gated_z=True, residual=x, out=x)
        return x

    def nbytes(self):
        return self.in_proj.nbytes() + self.out_proj.nbytes()


class AttnBlock:
    """mlx-lm NemotronH "*" block: x + o_proj(sdpa(q, k, v over the cache)), q|k|v from one
    concatenated 4-bit projection of norm(x); no positional encoding in this family."""

    def __init__(self, cfg: ModelConfig, init: _Init):
        D = cfg.hidden
        self.cfg = cfg
        self.norm_w = init.uniform(D)
        self.norm_w[0] = 0.0
        self.qkv = nn.QWeight(*init.q4(cfg.qkv_dim, D, 1.0 / math.sqrt(D)))
        QD = cfg.attn_heads * cfg.head_dim
        w, s, b = init.q4(D, QD, cfg.resid_scale / math.sqrt(QD))
        _zero_output_row0(w, s, b)
        self.o_proj = nn.QWeight(w, s, b)

    def rows(self, x, buf, kv: nn.KVCache, pos, status=None):
        B = x.shape[0]
        c = self.cfg
        qkv = nn.linear(x, self.qkv, norm=self.norm_w, eps=c.eps, out=buf["qkv"][:B])
        o = nn.attention(qkv, kv, pos, n_heads=c.attn_heads, n_kv_heads=c.kv_heads, head_dim=c.head_dim,
                         out=buf["att"][:B], workspace=buf["ws_attn"], status=status)
        nn.linear(o, self.o_proj, residual=x, out=x)
        return x

    def nbytes(self):
        return self.qkv.nbytes() + self.o_proj.nbytes()


class MoEBlock:
    """hsd/model.py:53-175 MoEBlock: router (bf16 gate, sigmoid scores + selection bias,
    top-k, normalised and scaled gains), the routed and shared 4-bit up projections with
    ReLU^2, and the down projection on the neuron-major layout over the live rows only
    (mode "sparse") or over every row with the same kernel (mode "dense", the dense-h
    control: bit-identical results), then the residual add."""

    def __init__(self, cfg: ModelConfig, init: _Init):
        D, E, F, FS = cfg.hidden, cfg.n_experts, cfg.moe_inter, cfg.shared_inter
        self.cfg = cfg
        self.norm_w = init.uniform(D)
        gate = init.bf16(E, D, std=1.0 / math.sqrt(D))
        gate[:, 0] = 0.0                                 # the bias channel does not steer the router
        self.gate = nn.QWeight(gate)
        self.trace = None
        self.e_bias = init.normal_f32(E, std=0.02)
        up_std = 1.0 / math.sqrt(D)
        self.w1, self.s1, self.b1 = init.q4(F, D, up_std, lead=(E,))
        self.sw1, self.ss1, self.sb1 = init.q4(FS, D, up_std)
        # the bias channel: input 0 of every up row has nibble 0, so W[j, 0] = b_j0 ~ -7.5 s
        # (negative): with xn[0] large the pre-activation gets a negative offset, which sets
        # the ReLU^2 zero fraction (real checkpoints have ~90 % zeros, hsd README)
        for w in (self.w1, self.sw1):
            w[..., 0] &= ~0xF
        # norm_w[0] scales xn[0] = norm_w[0] * c0 / rms(x): chosen by calibrate_sparsity
        self.norm_w[0] = 1.0
        live = max(1.0 - cfg.zero_frac, 0.02)
        dn_std = cfg.resid_scale / math.sqrt(F * live * 3.0)
        w, s, b = init.q4(D, F, dn_std, lead=(E,))
        _zero_output_row0(w, s, b)
        sw, ss, sb = init.q4(D, FS, dn_std)
        _zero_output_row0(sw, ss, sb)
        # neuron-major layout (the stock one is not kept: one resident layout, model.py:89-107)
        self.pw, self.ps, self.pb = layout.to_neuron_major(w, s, b)
        self.spw, self.sps, self.spb = layout.to_neuron_major(sw, ss, sb)
        del w, s, b, sw, ss, sb

    def rows(self, x, buf, dense=False, status=None):
        B = x.shape[0]
        c = self.cfg
        xn = buf["xn"][:B]
        logits = nn.linear(x, self.gate, norm=self.norm_w, eps=c.eps, out=buf["logits"][:B], xn_out=xn)
        if B <= 3:
            # the router's top-k fused into the up projections (a wavefront of every routed
            # workgroup ranks the experts), one launch fewer: 12.2 against 13.9 us at one row;
            # at three, since the top-k runs on DPP moves, the MTP-2 step takes 1.970 against
            # 1.977 ms (it was 28.7 against 25.1 us per layer with LDS shuffles)
            hcat, sel, gains = route_up_relu2(xn, logits, self.e_bias, self.w1, self.s1, self.b1, self.sw1,
                                              self.ss1, self.sb1, topk=c.topk, routed_scale=c.routed_scale,
                                              norm_topk=c.norm_topk, out=buf["hcat"][:B], sel=buf["sel"][:B],
                                              gains=buf["gains"][:B])
        else:
            # more rows: the router runs on its own first; same selection, same bits
            sel, gains = router_topk(logits, self.e_bias, topk=c.topk, routed_scale=c.routed_scale,
                                     norm_topk=c.norm_topk, sel=buf["sel"][:B], gains=buf["gains"][:B])
            hcat = up_relu2(xn, sel, self.w1, self.s1, self.b1, self.sw1, self.ss1, self.sb1, topk=c.topk,
                            out=buf["hcat"][:B])
        if self.trace is not None:                       # calibration / statistics only
            self.trace.append(float((hcat == 0).float().mean().item()))
        ws = buf["ws_down"]
        N.call("hsd_sparse_down_residual", N.ptr(hcat), N.DT_BF16, N.ptr(sel), N.ptr(gains),
               N.ptr(N.as_words(self.pw)), N.ptr(self.ps), N.ptr(self.pb), N.ptr(N.as_words(self.spw)),
               N.ptr(self.sps), N.ptr(self.spb), N.ptr(x), N.ptr(x), B, c.hidden, c.moe_inter, c.shared_inter, c.topk,
               c.n_experts, 1 if dense else 0, None, N.ptr(status), N.ptr(ws), ws.numel(), N.stream(x.device))
        return x

    # ---- the reference's per-block call surface (model.py:110-175) on fresh buffers: any
    # number of rows, results identical to rows() on the same rows
    def _front_packed(self, x):
        c = self.cfg
        x = N.contig(x)
        xn = torch.empty_like(x)
        logits = nn.linear(x, self.gate, norm=self.norm_w, eps=c.eps, xn_out=xn)
        sel, gains = router_topk(logits, self.e_bias, topk=c.topk, routed_scale=c.routed_scale, norm_topk=c.norm_topk)
        hcat = up_relu2(xn, sel, self.w1, self.s1, self.b1, self.sw1, self.ss1, self.sb1, topk=c.topk)
        return hcat, sel, gains

    def front(self, x):
        """model.py:110-121. x [B, D] bf16 -> (inds [B, topk] int32, scores [B, topk] f32,
        h [B, topk, F], hs [B, FS]) after ReLU^2 (views of one hcat block)."""
        c = self.cfg
        hcat, sel, gains = self._front_packed(x)
        B, KF = x.shape[0], c.topk * c.moe_inter
        return sel, gains[:, :c.topk], hcat[:, :KF].view(B, c.topk, c.moe_inter), hcat[:, KF:]

    def pack(self, inds, scores, h, hs):
        """model.py:123-129 -> (hcat [B, topk*F + FS], sel [B, topk] int32, gains [B, topk+1]
        f32: the scores, then 1 for the shared expert)."""
        B = h.shape[0]
        hcat = torch.cat([h.reshape(B, -1), hs.to(h.dtype)], dim=1).contiguous()
        gains = torch.cat([scores.float(), torch.ones((B, 1), dtype=torch.float32, device=h.device)], dim=1)
        return hcat, N.contig(inds.to(torch.int32)), gains.contiguous()

    def _down_residual(self, x, hcat, sel, gains, dense):
        c = self.cfg
        B = x.shape[0]
        out = N.contig(x).clone()
        nb = N.lib().hsd_sparse_down_workspace_bytes(B, c.hidden, c.moe_inter, c.shared_inter, c.topk)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=x.device)
        N.call("hsd_sparse_down_residual", N.ptr(hcat), N.DT_BF16, N.ptr(sel), N.ptr(gains),
               N.ptr(N.as_words(self.pw)), N.ptr(self.ps), N.ptr(self.pb), N.ptr(N.as_words(self.spw)),
               N.ptr(self.sps), N.ptr(self.spb), N.ptr(out), N.ptr(out), B, c.hidden, c.moe_inter, c.shared_inter,
               c.topk, c.n_experts, 1 if dense else 0, None, None, N.ptr(ws), ws.numel(), N.stream(x.device))
        return out

    def decode_sparse(self, x):
        """model.py:135-139: x [B, D] -> x + the MoE output, the down projection over the
        live rows of the neuron-major layout (a new tensor; x is not written)."""
        return self._down_residual(x, *self._front_packed(x), dense=False)

    def decode_dense(self, x):
        """model.py:132-133, the dense-h control: the same kernel over every row of the
        layout (the stock layout is not kept), bit-identical to decode_sparse."""
        return self._down_residual(x, *self._front_packed(x), dense=True)

    def prefill(self, x, mode="sparse"):
        """model.py:151-154."""
        return self.prefill_sparse(x) if mode == "sparse" else self.decode_dense(x)

    def prefill_sparse(self, x, tt=32):
        """model.py:156-175: x [T, D] -> x + the MoE output, the down projection as the
        grouped MFMA GEMM over each expert tile's union of live rows (tiles, unions and
        the GEMM on the device)."""
        from . import prefill as P
        c = self.cfg
        hcat, sel, gains = self._front_packed(x)
        tiles = P.build_tiles(sel, c.n_experts, tt)
        union = P.build_union(hcat, tiles[0], tiles[1], F=c.moe_inter, FS=c.shared_inter, topk=c.topk,
                              E=c.n_experts, tt=tt)
        y = P.sparse_down_prefill(hcat, sel, gains, self.pw, self.ps, self.pb, self.spw, self.sps, self.spb,
                                  F=c.moe_inter, FS=c.shared_inter, D=c.hidden, topk=c.topk, E=c.n_experts, tt=tt,
                                  tiles=tiles, union=union)
        return x + y.to(x.dtype)

    def nbytes(self):
        t = [self.gate.w, self.w1, self.s1, self.b1, self.sw1, self.ss1, self.sb1, self.pw, self.ps, self.pb,
             self.spw, self.sps, self.spb]
        return sum(a.numel() * a.element_size() for a in t)


class MTPHeadModule:
    """hsd/mtp.py:41-88 MTPHead: x = eh_proj(concat(rms_norm(embed(tok), enorm),
    rms_norm(h, hnorm))) -> attention block -> MoE block -> rms_norm(final_norm) -> the
    target's lm_head -> argmax. Its attention block keeps a KV cache over the rows the
    target has confirmed."""

    def __init__(self, cfg: ModelConfig, init: _Init):
        D = cfg.hidden
        self.enorm = init.uniform(D)
        self.enorm[0] = 1.0
        self.hnorm = init.uniform(D)
        self.hnorm[0] = 0.0
        eh = init.bf16(D, 2 * D, std=1.0 / math.sqrt(2 * D))
        # the head's residual stream keeps the bias channel too: output 0 copies the normed
        # embedding's channel 0 (the constant c0 over the embedding row's rms)
        eh[0] = 0.0
        eh[0, 0] = 1.0
        self.eh_proj = nn.QWeight(eh)
        self.attn = AttnBlock(cfg, init)
        self.moe = MoEBlock(cfg, init)
        self.final_norm = init.uniform(D)
        self.final_norm[0] = 0.0

    def nbytes(self):
        return self.eh_proj.nbytes() + self.attn.nbytes() + self.moe.nbytes()


# ------------------------------------------------------------------ caches
class ModelCache:
    """Every layer's cache plus the sequence state (hsd_native SEQ_* indices): attention
    KV caches whose length is seq[POS], Mamba checkpoint rings sharing the index seq[CUR],
    and the MTP head's KV cache (length seq[HEAD_POS])."""

    def __init__(self, model: "NemotronModel", cap=4096):
        c, dev = model.cfg, model.device
        self.seq = torch.zeros(N.SEQ_LEN, dtype=torch.int32, device=dev)
        # HSD_STATUS_* bits the kernels OR in (an attention cache overflow, a corrupt ring
        # index, a token or expert id out of range); checked after every prefill and step
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.cur = self.seq[N.SEQ_CUR:N.SEQ_CUR + 1]
        self.pos = self.seq[N.SEQ_POS:N.SEQ_POS + 1]
        self.head_pos = self.seq[N.SEQ_HEAD_POS:N.SEQ_HEAD_POS + 1]
        self.head_pos2 = self.seq[N.SEQ_HEAD_POS2:N.SEQ_HEAD_POS2 + 1]
        self.layers = []
        for t, blk in zip(c.pattern, model.blocks):
            if t == "M":
                self.layers.append(M.MambaCache(blk.mixer, dev, nslab=NSLAB, cur=self.cur))
            elif t == "*":
                self.layers.append(nn.KVCache(c.kv_heads, c.max_seq, dev, c.head_dim))
            else:
                self.layers.append(None)
        self.head_kv = nn.KVCache(c.kv_heads, c.max_seq, dev, c.head_dim) if model.mtp is not None else None
        self.out_tokens = torch.zeros(cap, dtype=torch.int32, device=dev)
        self.cap = cap

    def state(self):
        return self.seq.cpu().tolist()

    def check_status(self, where):
        """Raises HSDError when a kernel has flagged this cache's status word (reads one
        int back: call it after a synchronise, not inside a captured step)."""
        st = int(self.status.item())
        if st:
            why = [n for bit, n in ((N.STATUS_BAD_EXPERT, "an expert id out of range"),
                                    (N.STATUS_BAD_STATE, "an attention cache overflow or a corrupt Mamba ring index"),
                                    (N.STATUS_BAD_TOKEN, "a token id out of range")) if st & bit]
            raise N.HSDError(f"{where}: device status {st} ({'; '.join(why)})")


# ------------------------------------------------------------------ the model
class NemotronModel:
    """hsd/model.py:178-443 NemotronModel on libhsd. `mode` is "sparse" or "dense" (the MoE
    down projection over the live rows, or over every row with the same kernel)."""

    def __init__(self, cfg: ModelConfig | None = None, mode="sparse", seed=0, device="cuda:0", verbose=False,
                 calibrate=True):
        self.cfg = cfg = cfg or ModelConfig()
        self.device = torch.device(device)
        if mode not in ("sparse", "dense"):
            raise ValueError(mode)
        self.mode = mode
        t0 = time.time()
        init = _Init(seed, self.device)
        D, V = cfg.hidden, cfg.vocab
        # embedding: ~N(0, 1)-sized entries; channel 0 (the bias channel) is the constant c0
        ew, es, eb = init.q4(V, D, 1.0)
        ew[:, 0] = (ew[:, 0] & ~0xF) | 0xF                        # nibble 15 at input 0
        es[:, 0] = 0.25
        eb[:, 0] = -1.875                                         # group 0: s (q - 7.5)
        self.embedding = nn.QWeight(ew, es, eb)
        self.c0 = 15 * 0.25 - 1.875
        self.blocks = []
        for t in cfg.pattern:
            self.blocks.append({"M": MambaBlock, "E": MoEBlock, "*": AttnBlock}[t](cfg, init))
        self.norm_f = init.uniform(D)
        self.norm_f[0] = 0.0
        self.lm_head = nn.QWeight(*init.q4(V, D, 1.0 / math.sqrt(D)))
        self.mtp = MTPHeadModule(cfg, init) if cfg.mtp else None
        self.slots = nn.argmax_slots(V)
        self._bufs = {B: self._make_buffers(B) for B in ROWS}
        self.zero_frac_measured = None
        if calibrate:
            self.calibrate_sparsity()
        self.load_seconds = time.time() - t0
        if verbose:
            print(f"model: {len(cfg.pattern)} layers, {self.nbytes() / 1e9:.2f} GB of weights, "
                  f"{self.load_seconds:.1f} s", flush=True)

    # ---- buffers (preallocated per row count so that steps capture into graphs)
    def _make_buffers(self, B):
        c, dev = self.cfg, self.device
        e = lambda *s, dt=torch.bfloat16: torch.zeros(s, dtype=dt, device=dev)
        ws_down = N.lib().hsd_sparse_down_workspace_bytes(B, c.hidden, c.moe_inter, c.shared_inter, c.topk)
        ws_attn = N.lib().hsd_attn_workspace_bytes(B, c.attn_heads, c.max_seq)
        return dict(x=e(B, c.hidden), xn=e(B, c.hidden), proj=e(B, c.in_proj_dim),
                    y_pre=e(B, c.mamba_inner + c.mamba_inner // 16, dt=torch.float32), qkv=e(B, c.qkv_dim),
                    att=e(B, c.attn_heads * c.head_dim), logits=e(B, c.n_experts),
                    hcat=e(B, c.topk * c.moe_inter + c.shared_inter), sel=e(B, c.topk, dt=torch.int32),
                    gains=e(B, c.topk + 1, dt=torch.float32),
                    ws_down=e(ws_down, dt=torch.uint8), ws_attn=e(ws_attn, dt=torch.uint8),
                    keys=e(B, self.slots, dt=torch.int64), ids=e(max(B, 4), dt=torch.int32),
                    # MTP head
                    pair=e(B, 2 * c.hidden), emb=e(B, c.hidden), hx=e(B, c.hidden), hn=e(B, c.hidden),
                    pend=e(4, dt=torch.int32), d1=e(4, dt=torch.int32), keys2=e(1, self.slots, dt=torch.int64),
                    h2=e(1, c.hidden), hn1=e(1, c.hidden),
                    keys1=e(1, self.slots, dt=torch.int64),
                    # the head's residual rows and attention output side by side, so one
                    # row selection takes both
                    hcomb=e(B, c.hidden + c.attn_heads * c.head_dim))

    def moe_blocks(self):
        out = [b for t, b in zip(self.cfg.pattern, self.blocks) if t == "E"]
        if self.mtp is not None:
            out.append(self.mtp.moe)
        return out

    def calibrate_sparsity(self, n_tokens=48, iters=3, seed=1234):
        """Sets each MoE block's norm weight on the bias channel so that its ReLU^2
        activations have about cfg.zero_frac exact zeros (the synthetic model's stand-in
        for a trained checkpoint's activation sparsity). The offset the bias channel adds
        to every up-projection pre-activation scales with that weight; its zero fraction
        z behaves like Phi(k w), so w is rescaled by Phi^-1(target) / Phi^-1(z) from
        eager prefills of a random prompt. Returns the measured zero fraction per MoE
        block (target blocks, then the MTP head's)."""
        from statistics import NormalDist
        nd = NormalDist()
        target = min(max(self.cfg.zero_frac, 0.51), 0.995)
        blocks = self.moe_blocks()
        # first guess: offset = -7.5 s (mean s = std / 4.61) * xn0, xn0 ~ w0 * c0 / rms
        D = self.cfg.hidden
        w0 = nd.inv_cdf(target) / (7.5 / 4.61 / math.sqrt(D) * self.c0)
        for b in blocks:
            b.norm_w[0] = w0
        rng = np.random.default_rng(seed)
        prompt = rng.integers(0, self.cfg.vocab, n_tokens).astype(np.int32)
        z = []
        for it in range(iters + 1):
            for b in blocks:
                b.trace = []
            cache = self.make_cache(cap=4)
            self.prefill(prompt, cache, with_head=self.mtp is not None, graph=False)
            torch.cuda.synchronize(self.device)
            z = [float(np.mean(b.trace)) for b in blocks]
            for b in blocks:
                b.trace = None
            if it == iters:
                break
            for b, zb in zip(blocks, z):
                zb = min(max(zb, 0.52), 0.999)
                w = float(b.norm_w[0].float().item())
                b.norm_w[0] = w * min(max(nd.inv_cdf(target) / nd.inv_cdf(zb), 0.25), 4.0)
            del cache
        self.zero_frac_measured = z
        return z

    def nbytes(self):
        n = self.embedding.nbytes() + self.lm_head.nbytes()
        n += sum(b.nbytes() for b in self.blocks)
        if self.mtp is not None:
            n += self.mtp.nbytes()
        return n

    def make_cache(self, cap=4096):
        return ModelCache(self, cap)

    def set_mode(self, mode):
        if mode not in ("sparse", "dense"):
            raise ValueError(mode)
        self.mode = mode

    # ---- pieces shared with the MTP head (model.py:222-230)
    def embed(self, ids, out=None, status=None):
        return nn.embed(ids, self.embedding, out=out, status=status)

    # ---- the stack
    def layers(self, x, buf, cache: ModelCache):
        """x [B, D] through every block in place; rows at positions POS .. POS+B-1."""
        dense = self.mode == "dense"
        st = cache.status
        for t, blk, lc in zip(self.cfg.pattern, self.blocks, cache.layers):
            if t == "M":
                blk.rows(x, buf, lc, status=st)
            elif t == "*":
                blk.rows(x, buf, lc, cache.pos, status=st)
            else:
                blk.rows(x, buf, dense=dense, status=st)
        return x

    def head_keys(self, x, buf, keys, norm=None):
        """lm_head(rms_norm(x)) -> the per-workgroup argmax keys (model.py:229-230, 419)."""
        nn.linear(x, self.lm_head, norm=self.norm_f if norm is None else norm, eps=self.cfg.eps, argmax_keys=keys)
        return keys

    def logits(self, x, norm=None):
        """bf16 logits lm_head(rms_norm(x)) [B, V] (tests and debugging)."""
        keys = torch.empty((x.shape[0], self.slots), dtype=torch.int64, device=x.device)
        out = torch.empty((x.shape[0], self.cfg.vocab), dtype=torch.bfloat16, device=x.device)
        nn.linear(x, self.lm_head, norm=self.norm_f if norm is None else norm, eps=self.cfg.eps, argmax_keys=keys,
                  out=out)
        return out

    # ---- the MTP head forward (mtp.py:74-88)
    def mtp_rows(self, h, toks, buf, kv: nn.KVCache, pos, keys=None, status=None, chain=None, select=None):
        """Head rows: h [B, D] (the target's pre-norm hidden), toks [B] int32 (the token
        after each row's position) at positions pos .. pos+B-1 of the head's KV cache kv.
        Leaves the normed hidden rows in buf["hn"] and (with keys) the argmax keys of the
        head's logits. chain = (keys, seq, d1): the chained call, its token the argmax of
        those keys and h the selected row's normed hidden row (nn.head_input).
        select = (seq, buf1): only row R - 1 (R from seq) goes on past the attention: every
        row enters the head's KV cache, but only that row's prediction is a draft
        (model.py:408-411), so o_proj and the MoE block run on it alone (buf1's one-row
        buffers) and the row [1, D] is returned."""
        B = h.shape[0]
        hd, c = self.mtp, self.cfg
        # the token embedding and the pair norm in one launch
        pair = nn.head_input(toks, h, self.embedding, hd.enorm, hd.hnorm, eps=c.eps, out=buf["pair"][:B],
                             status=status, chain=chain)
        if select is not None:
            seq, b1 = select
            D, a = c.hidden, hd.attn
            comb = buf["hcomb"][:B]
            x = nn.linear(pair, hd.eh_proj, out=comb[:, :D])
            qkv = nn.linear(x, a.qkv, norm=a.norm_w, eps=c.eps, out=buf["qkv"][:B])
            nn.attention(qkv, kv, pos, n_heads=c.attn_heads, n_kv_heads=c.kv_heads, head_dim=c.head_dim,
                         out=comb[:, D:], workspace=buf["ws_attn"], status=status)
            one = b1["hcomb"]
            N.call("hsd_seq_select_row", N.ptr(comb), comb.stride(0), N.ptr(seq), N.ptr(one), comb.shape[1],
                   N.stream(self.device))
            x1 = one[:, :D]
            nn.linear(one[:, D:], a.o_proj, residual=x1, out=x1)
            hd.moe.rows(x1, b1, dense=self.mode == "dense", status=status)
            return x1
        x = nn.linear(pair, hd.eh_proj, out=buf["hx"][:B])
        hd.attn.rows(x, buf, kv, pos, status=status)
        hd.moe.rows(x, buf, dense=self.mode == "dense", status=status)
        if keys is not None:
            nn.linear(x, self.lm_head, norm=hd.final_norm, eps=c.eps, argmax_keys=keys, xn_out=buf["hn"][:B])
        return x

    # ---- prefill (model.py:259-279), in steps of 3 rows through the decode kernels
    def _prefill_step(self, prompt_dev, T, cache, with_head):
        buf = self._bufs[3]
        ids = buf["ids"][:3]
        N.call("hsd_gather_tokens", N.ptr(prompt_dev), T, N.ptr(cache.seq), 0, 3, N.ptr(ids), N.stream(self.device))
        x = self.embed(ids, out=buf["x"], status=cache.status)
        self.layers(x, buf, cache)
        if with_head:
            pend = buf["pend"][:3]
            N.call("hsd_gather_tokens", N.ptr(prompt_dev), T, N.ptr(cache.seq), 1, 3, N.ptr(pend),
                   N.stream(self.device))
            self.mtp_rows(x, pend, buf, cache.head_kv, cache.head_pos, status=cache.status)
        N.call("hsd_prefill_advance", N.ptr(cache.seq), T, 3, NSLAB, N.stream(self.device))

    def prefill(self, tokens, cache: ModelCache, with_head=None, graph=True):
        """tokens [T] (host ints or a tensor) -> the residual stream of the last position
        [1, D] (pre norm_f), with every cache advanced by T rows (and, with the MTP head,
        its cache holding the rows (h_p, tok_{p+1}), p < T-1). The steps of 3 rows replay
        one captured graph."""
        with_head = (self.mtp is not None) if with_head is None else with_head
        prompt = torch.as_tensor(tokens, dtype=torch.int32).to(self.device)
        T = int(prompt.numel())
        nsteps = (T + 2) // 3
        if T < 1 or 3 * nsteps > self.cfg.max_seq:
            # the last 3-row step writes attention rows up to 3 * nsteps - 1
            raise N.HSDError(f"a {T}-token prompt needs {3 * nsteps} attention cache rows (3-row prefill steps); "
                             f"max_seq is {self.cfg.max_seq}")
        if graph and nsteps > 2:
            g = self._capture(lambda: self._prefill_step(prompt, T, cache, with_head))
            for _ in range(nsteps):
                g.replay()
            torch.cuda.synchronize(self.device)
            del g
        else:
            for _ in range(nsteps):
                self._prefill_step(prompt, T, cache, with_head)
        # the last prompt row: row (T - 1) % 3 of the last step
        r = (T - 1) % 3
        return self._bufs[3]["x"][r:r + 1]

    def _capture(self, fn, keep_graph=False):
        """A graph of fn() (one step; it reads and advances the sequence state on the
        device, so it is captured without a warm-up run: every buffer is preallocated and
        nothing allocates inside). The graph is bound to the caches fn uses; the caller
        keeps it only while they live. keep_graph: the hipGraph_t stays readable
        (raw_cuda_graph()) until the graph is instantiated."""
        g = torch.cuda.CUDAGraph(keep_graph=keep_graph)
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s), N.capture_guard():
            with torch.cuda.graph(g, stream=s):
                fn()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return g

    # ---- plain decode (model.py:281-323)
    def _decode_step(self, cache):
        buf = self._bufs[1]
        x = self.embed(cache.seq[N.SEQ_TOK:N.SEQ_TOK + 1], out=buf["x"], status=cache.status)
        self.layers(x, buf, cache)
        self.head_keys(x, buf, buf["keys"])
        N.call("hsd_decode_advance", N.ptr(buf["keys"]), self.slots, N.ptr(cache.seq), N.ptr(cache.out_tokens),
               cache.cap, NSLAB, N.stream(self.device))

    def step(self, x, cache):
        """One decode step on x [1, D] through every block (model.py:281-288)."""
        return self.layers(x, self._bufs[1], cache)

    def _first_token(self, x_last, cache):
        """tok0 = argmax(lm_head(norm_f(h_{T-1}))): out_tokens[0], N = 1, TOK = tok0."""
        buf = self._bufs[1]
        buf["x"].copy_(x_last)
        self.head_keys(buf["x"], buf, buf["keys"])
        # the advance of a decode step, then POS / CUR / STEPS back: the prompt's rows are
        # already in the caches
        st = N.stream(self.device)
        N.call("hsd_decode_advance", N.ptr(buf["keys"]), self.slots, N.ptr(cache.seq), N.ptr(cache.out_tokens),
               cache.cap, NSLAB, st)
        N.call("hsd_seq_rollback", N.ptr(cache.seq), 1, NSLAB, st)
        N.call("hsd_seq_add", N.ptr(cache.seq), N.SEQ_STEPS, -1, st)

    def session(self, prompt, *, mtp=False, cap=4096, script=None, accepts=None, graph=True):
        """A generation after its prompt: the prompt prefilled (and the first token chosen),
        then `step(n)` replays n decode steps (mtp=False) or n MTP steps (mtp=True: draft,
        verify 3 rows, accept, roll back) from one captured graph with no host round trip.
        With `script` (the true continuation) and `accepts` (accepted drafts per step) the
        drafts are forced."""
        return Session(self, prompt, mtp=mtp, cap=cap, script=script, accepts=accepts, graph=graph)

    def generate(self, prompt, max_tokens=128, cache=None, graph=True):
        """Greedy generation (model.py:291-323). Yields (token, stats) per token; stats is
        None except on the last yield. The decode steps replay one captured graph with no
        host round trip; the tokens are read back once at the end."""
        del cache
        s = self.session(prompt, cap=max(max_tokens, 1), graph=graph)
        s.step(max_tokens - 1)
        out = s.tokens(max_tokens)
        stats = self._stats(len(prompt), s.prompt_s, len(out), s.decode_s, out)
        for i, t in enumerate(out):
            yield t, (stats if i == len(out) - 1 else None)

    def _stats(self, T, prompt_s, n, dec_s, out, **extra):
        return dict(mode=self.mode, prompt_tokens=T, prompt_s=prompt_s, prompt_tps=T / prompt_s, gen_tokens=n,
                    decode_s=dec_s, decode_tps=(n - 1) / dec_s if n > 1 else float("nan"),
                    ms_per_token=1e3 * dec_s / max(n - 1, 1),
                    peak_gb=torch.cuda.max_memory_allocated(self.device) / 1e9, tokens=out, **extra)

    # ---- verify / rollback (model.py:333-356)
    def verify_step(self, x, cache):
        """x [B, D] (B <= 3 consecutive positions) through every layer in one pass; every
        cache advanced by B rows. Returns the final residual stream [B, D]."""
        B = x.shape[0]
        buf = self._bufs[3]
        xb = buf["x"][:B]
        if xb.data_ptr() != x.data_ptr():
            xb.copy_(x)
        self.layers(xb, buf, cache)
        N.call("hsd_seq_add", N.ptr(cache.seq), N.SEQ_POS, B, N.stream(self.device))
        N.call("hsd_mamba_select_row", N.ptr(cache.cur), None, B, B, NSLAB, None, N.stream(self.device))
        return xb

    def rollback(self, cache, n_keep, B):
        """Undo a verify_step of B rows beyond its first n_keep (attention caches trimmed,
        Mamba rings back to the checkpoint of row n_keep - 1)."""
        if n_keep == B:
            return
        N.call("hsd_seq_rollback", N.ptr(cache.seq), B - n_keep, NSLAB, N.stream(self.device))

    # ---- MTP speculative decoding (model.py:366-443)
    def _mtp_step(self, cache, script=None, accepts=None):
        b3, b1 = self._bufs[3], self._bufs[1]
        c = self.cfg
        st = N.stream(self.device)
        # the head over the rows the last verify confirmed (R of them valid); only row R-1's
        # prediction is a draft (model.py:408-411), so lm_head runs on that row alone
        x1 = self.mtp_rows(b3["x"], b3["pend"][:3], b3, cache.head_kv, cache.head_pos, status=cache.status,
                           select=(cache.seq, b1))
        nn.linear(x1, self.lm_head, norm=self.mtp.final_norm, eps=c.eps, argmax_keys=b1["keys1"],
                  xn_out=b1["hn1"])
        # the chained call on its own normed hidden row (mtp.py, model.py:411-413); its input
        # launch also takes the first draft from keys1 (d1) and the cache row (HEAD_POS2)
        self.mtp_rows(b1["hn1"], None, b1, cache.head_kv, cache.head_pos2, keys=b1["keys2"], status=cache.status,
                      chain=(b1["keys1"], cache.seq, b3["d1"]))
        # verify [tok, d1, d2] in one pass of 3 rows, then accept and roll back on the device;
        # one launch writes the ids and their embedding rows
        ids = b3["ids"]
        emb = self.embedding
        N.call("hsd_verify_input", N.ptr(b3["d1"]), N.ptr(b1["keys2"]), self.slots, 2, N.ptr(cache.seq),
               N.ptr(script), 0 if script is None else script.numel(), N.ptr(accepts),
               0 if accepts is None else accepts.numel(), c.vocab, N.ptr(emb.w), N.ptr(emb.scales),
               N.ptr(emb.biases), c.hidden, N.ptr(ids), N.ptr(b3["x"]), b3["x"].stride(0), N.ptr(cache.status), st)
        x = b3["x"][:3]
        self.layers(x, b3, cache)
        self.head_keys(x, b3, b3["keys"])
        N.call("hsd_spec_accept", N.ptr(b3["keys"]), b3["keys"].stride(0), self.slots, 2, N.ptr(ids),
               N.ptr(cache.seq), N.ptr(cache.out_tokens), cache.cap, NSLAB, N.ptr(b3["pend"]), None, st)

    def generate_mtp(self, prompt, mtp=None, n_draft=2, max_tokens=128, script=None, accepts=None, graph=True):
        """Greedy speculative decoding with the MTP head (model.py:366-443). Per step: the
        head over the rows the last verify confirmed, chained once for the second draft;
        the target verifies [token, draft1, draft2] in one pass of 3 rows; the greedy
        acceptance, the emitted tokens and the rollback of every cache happen on the device.
        With `script` (the true continuation) and `accepts` (accepted drafts per step) the
        drafts are forced (scripted acceptance). Yields (token, stats) like generate."""
        if n_draft != 2 or self.mtp is None:
            raise N.HSDError("generate_mtp runs the one-layer MTP head with 2 drafts")
        del mtp                                   # the head is the model's own (self.mtp)
        s = self.session(prompt, mtp=True, cap=max_tokens + 4, script=script, accepts=accepts, graph=graph)
        if accepts is not None:
            # the scripted counts fix how many steps produce max_tokens
            n, need = 1, 0
            while n < max_tokens:
                n += int(accepts[min(need, len(accepts) - 1)]) + 1
                need += 1
            s.step(need)
        else:
            while s.emitted() < max_tokens:
                s.step(4)
        seq = s.state()
        out = s.tokens(max_tokens)
        acc_mean = seq[N.SEQ_ACC_SUM] / max(seq[N.SEQ_STEPS], 1)
        stats = self._stats(len(prompt), s.prompt_s, len(out), s.decode_s, out,
                            spec=dict(kind="mtp", n_draft=2, steps=seq[N.SEQ_STEPS], accepted_mean=acc_mean,
                                      tokens_per_step=(len(out) - 1) / max(seq[N.SEQ_STEPS], 1)))
        for i, t in enumerate(out):
            yield t, (stats if i == len(out) - 1 else None)


class Session:
    """One generation's caches after the prompt, and its captured step graph."""

    def __init__(self, model: NemotronModel, prompt, *, mtp, cap, script, accepts, graph):
        self.m = model
        self.mtp = mtp
        dev = model.device
        if mtp and model.mtp is None:
            raise N.HSDError("an MTP session needs the model's MTP head")
        self.prompt_len = T = len(prompt)
        self.max_seq = model.cfg.max_seq
        # attention cache rows: the prompt's (3-row prefill steps write up to 3 ceil(T / 3)),
        # then one per generated token and the two draft rows of a verify beyond the last
        if 3 * ((T + 2) // 3) > self.max_seq or T + cap + 2 > self.max_seq:
            raise N.HSDError(f"a {T}-token prompt and {cap} generated tokens need {max(3 * ((T + 2) // 3), T + cap + 2)} "
                             f"attention cache rows; max_seq is {self.max_seq}")
        self.cache = cache = model.make_cache(cap=cap + 4)
        self.script = None if script is None else torch.as_tensor(script, dtype=torch.int32).to(dev)
        self.accepts = None if accepts is None else torch.as_tensor(accepts, dtype=torch.int32).to(dev)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        x_last = model.prefill(prompt, cache, with_head=mtp, graph=graph)
        model._first_token(x_last, cache)
        if mtp:
            # the head's pending row: (h_{T-1}, tok0)
            b3 = model._bufs[3]
            b3["x"][0].copy_(x_last[0])
            b3["pend"][0:1].copy_(cache.seq[N.SEQ_TOK:N.SEQ_TOK + 1])
            N.call("hsd_seq_add", N.ptr(cache.seq), N.SEQ_R, 1, N.stream(dev))
        torch.cuda.synchronize(dev)
        self.prompt_s = time.perf_counter() - t0
        cache.check_status("prefill")
        self.n_bound = 1                  # an upper bound of the emitted count (exact after emitted())
        # the step closes over the model and the caches, not over the session: a session
        # dropped by its caller (and the graph it owns) is freed at once, not by the cycle
        # collector
        if mtp:
            script, accepts = self.script, self.accepts
            fn = lambda: model._mtp_step(cache, script, accepts)
        else:
            fn = lambda: model._decode_step(cache)
        self.step_fn = fn
        self._run = model._capture(fn).replay if graph else fn
        self.decode_s = 0.0
        self.steps = 0

    def step(self, n=1):
        """n steps, timed with events on the stream they run on (after a synchronise);
        returns their seconds."""
        if n <= 0:
            return 0.0
        per = 3 if self.mtp else 1
        if self.prompt_len + self.n_bound + per * n + 1 > self.max_seq:
            # a step's rows sit at POS = T + emitted - 1 onwards (up to 3 of them): refresh the
            # bound from the device before refusing
            self.emitted()
            if self.prompt_len + self.n_bound + per * n + 1 > self.max_seq:
                raise N.HSDError(f"{n} more steps could pass the attention cache's {self.max_seq} rows "
                                 f"(prompt {self.prompt_len}, up to {self.n_bound} tokens emitted)")
        dev = self.m.device
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            self._run()
        e1.record()
        torch.cuda.synchronize(dev)
        sec = e0.elapsed_time(e1) * 1e-3
        self.decode_s += sec
        self.steps += n
        self.n_bound += per * n
        self.cache.check_status("decode step")
        return sec

    def state(self):
        return self.cache.state()

    def emitted(self):
        self.n_bound = int(self.cache.seq[N.SEQ_N].item())
        return self.n_bound

    def tokens(self, limit=None):
        n = min(self.emitted(), self.cache.cap)
        if limit is not None:
            n = min(n, limit)
        return self.cache.out_tokens[:n].cpu().tolist()
