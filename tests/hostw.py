"""Host copies of a hsd.model block's weights in the oracle's conventions (bf16 bits as
uint16, 4-bit words as uint32, float32 for the f32 parameters)."""
import numpy as np

from hsd import synth as S


def _u32(t):
    return S.to_host(t).view(np.uint32)


def mamba_block(blk):
    m = blk.mixer
    return dict(norm_w=S.to_host(blk.norm_w), in_w=_u32(blk.in_proj.w), in_s=S.to_host(blk.in_proj.scales),
                in_b=S.to_host(blk.in_proj.biases), out_w=_u32(blk.out_proj.w), out_s=S.to_host(blk.out_proj.scales),
                out_b=S.to_host(blk.out_proj.biases), conv_w=m.conv_w.float().cpu().numpy(),
                conv_b=m.conv_b.float().cpu().numpy(), A_log=m.A_log.cpu().numpy(), dt_bias=m.dt_bias.cpu().numpy(),
                D=m.D.cpu().numpy(), gnorm_w=S.to_host(m.norm_w))


def attn_block(blk):
    return dict(norm_w=S.to_host(blk.norm_w), qkv_w=_u32(blk.qkv.w), qkv_s=S.to_host(blk.qkv.scales),
                qkv_b=S.to_host(blk.qkv.biases), o_w=_u32(blk.o_proj.w), o_s=S.to_host(blk.o_proj.scales),
                o_b=S.to_host(blk.o_proj.biases))


def moe_block(blk):
    return dict(norm_w=S.to_host(blk.norm_w), gate=S.to_host(blk.gate.w), e_bias=blk.e_bias.cpu().numpy(),
                w1=_u32(blk.w1), s1=S.to_host(blk.s1), b1=S.to_host(blk.b1), sw1=_u32(blk.sw1),
                ss1=S.to_host(blk.ss1), sb1=S.to_host(blk.sb1), pw=_u32(blk.pw), ps=S.to_host(blk.ps),
                pb=S.to_host(blk.pb), spw=_u32(blk.spw), sps=S.to_host(blk.sps), spb=S.to_host(blk.spb))


def model_blocks(model):
    fn = {"M": mamba_block, "*": attn_block, "E": moe_block}
    return [fn[t](b) for t, b in zip(model.cfg.pattern, model.blocks)]
