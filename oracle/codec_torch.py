"""TEST INFRASTRUCTURE ONLY: the reference codec restated in torch CPU ops.

A second restatement beside the scalar C oracle (tests cross-check the two),
and the timed CPU baseline of bench.py: it follows the op
sequence of usaf/quantization.py:47-85 and :107-132 with torch's own CPU
kernels (amin/amax, true division, round-half-even, fp16 tensor arithmetic),
so a transcription slip in either restatement shows up as a mismatch.
"""
import torch


def quantize_opseq(tensor: torch.Tensor, group_size: int = 128):
    x = tensor.contiguous().flatten().float()                      # :47
    numel = x.numel()
    egs = min(group_size, numel)                                  # :50
    G = (numel + egs - 1) // egs                                  # :51
    if G * egs > numel:
        x = torch.cat([x, torch.zeros(G * egs - numel, dtype=x.dtype)])  # :54-55
    x2 = x.view(G, egs)
    mn = x2.amin(dim=1, keepdim=True)                             # :59
    mx = x2.amax(dim=1, keepdim=True)                             # :60
    scale = ((mx - mn) / 15.0).clamp_min(1e-12)                   # :62-63
    q = ((x2 - mn) / scale).round().clamp(0, 15).to(torch.uint8)  # :66-68
    even = q[:, 0::2]                                             # :74
    odd = torch.zeros_like(even)                                  # :75
    if egs > 1:
        odd[:, : q[:, 1::2].shape[1]] = q[:, 1::2]                # :77
    packed = (even | (odd << 4)).view(torch.int8)                 # :79-80
    return packed, scale.squeeze(1).half(), mn.squeeze(1).half()  # :82-83


def dequant_opseq(q_int4: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, shape, group_size=128):
    G, pb = q_int4.shape                                          # :107-108
    raw = q_int4.to(torch.uint8)                                  # :110
    inter = torch.empty((G, pb * 2), dtype=torch.uint8)           # :115
    inter[:, 0::2] = raw & 0x0F                                   # :111, :116
    inter[:, 1::2] = (raw >> 4) & 0x0F                            # :112, :117
    numel = 1
    for s in shape:
        numel *= int(s)
    egs = min(group_size, numel)                                  # :124
    q = inter.flatten()[: G * egs].view(G, egs).to(torch.float16) # :127
    x = q * scale.half().unsqueeze(1) + zero.half().unsqueeze(1)  # :129
    return x.flatten()[:numel].view(shape)                        # :132
