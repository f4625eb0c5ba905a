"""Algorithmic FLOP count of one SDXL UNet forward, by kernel class.

2 FLOPs per multiply-add; padding, recomputation and the elementwise /
normalisation work are not counted.  For the SDXL configuration at B=2 and
a 128x128 latent this gives 13.522 TFLOP: convs 3.246 (3x3 3.112, 1x1
shortcuts 0.134), attention 1.568 (self 1.503, cross 0.065), linears 8.708.
"""


def unet_step_flops(B=2, H=128, W=128, C=(320, 640, 1280), depth=(0, 2, 10), ctx=77,
                    cross=2048, text_dim=1280, id_dim=256, cin=4, cout=4):
    C0, C1, C2 = C
    T = 4 * C0
    res = {"conv3": 0.0, "conv1": 0.0, "attn_self": 0.0, "attn_cross": 0.0, "linear": 0.0,
           "small": 0.0}

    def conv3(HW, ci, co):
        res["conv3"] += 2.0 * B * HW * co * 9 * ci

    def resnet(HW, ci, co):
        conv3(HW, ci, co)
        conv3(HW, co, co)
        res["small"] += 2.0 * B * T * co
        if ci != co:
            res["conv1"] += 2.0 * B * HW * co * ci

    def t2d(HW, c, d):
        M = B * HW
        res["linear"] += 2 * 2.0 * M * c * c  # proj_in, proj_out
        for _ in range(d):
            res["linear"] += 2.0 * M * c * c * (3 + 1 + 1 + 1 + 8 + 4)
            res["linear"] += 2 * 2.0 * B * ctx * cross * c  # cross K, V
            res["attn_self"] += 4.0 * B * HW * HW * c
            res["attn_cross"] += 4.0 * B * HW * ctx * c

    HW = [H * W, (H // 2) * (W // 2), (H // 4) * (W // 4)]
    Cs = [C0, C1, C2]
    res["small"] += 2.0 * B * (T * C0 + T * T + T * (text_dim + 6 * id_dim) + T * T)
    conv3(HW[0], cin, C0)
    prev = C0
    skips = [C0]
    for lv in range(3):
        for r in range(2):
            resnet(HW[lv], prev if r == 0 else Cs[lv], Cs[lv])
            if depth[lv]:
                t2d(HW[lv], Cs[lv], depth[lv])
            skips.append(Cs[lv])
        prev = Cs[lv]
        if lv < 2:
            conv3(HW[lv + 1], Cs[lv], Cs[lv])  # stride-2 conv at the lower resolution
            skips.append(Cs[lv])
    resnet(HW[2], C2, C2)
    t2d(HW[2], C2, depth[2])
    resnet(HW[2], C2, C2)
    cur = C2
    for u in range(3):
        lv = 2 - u
        for r in range(3):
            resnet(HW[lv], cur + skips.pop(), Cs[lv])
            cur = Cs[lv]
            if depth[lv]:
                t2d(HW[lv], Cs[lv], depth[lv])
        if u < 2:
            conv3(HW[lv - 1], Cs[lv], Cs[lv])  # upsample conv at 2x resolution
    conv3(HW[0], C0, cout)
    out = dict(res)
    out["conv"] = res["conv3"] + res["conv1"]
    out["attention"] = res["attn_self"] + res["attn_cross"]
    out["total"] = out["conv"] + out["attention"] + res["linear"]
    return out


def mid_block_flops(B=2, HW=32 * 32, C=1280, depth=10, ctx=77, cross=2048):
    """FLOPs of mid_block (resnet + Transformer2D + resnet) for the CPU sample."""
    f = 2 * 2 * (2.0 * B * HW * C * 9 * C)
    M = B * HW
    f += 2 * 2.0 * M * C * C
    f += depth * (2.0 * M * C * C * 18 + 2 * 2.0 * B * ctx * cross * C + 4.0 * B * HW * HW * C
                  + 4.0 * B * HW * ctx * C)
    return f
