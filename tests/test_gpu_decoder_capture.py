"""A stack of Gemma 4 decoder layers at the 26B-A4B shape, everything but attention, captured into one
HIP graph: the capture safety the reference relies on when it captures whole decoder steps
(flide/backbones/gemma4/graphs.py:193-215), with this MoE layer inside.

Each layer follows flide/backbones/gemma4/fused.py:208-229 (the `ple`-less branch):
  d = attention output (here a plain product of the layer input: attention is not on this path)
  h, x = sandwich(d, h, post_attention_layernorm, w2=pre_feedforward_layernorm)    (torch glue)
  dense = down(geglu(gate_up(x)))                                                  (torch products)
  logits, x2 = router_norm(h, ...); top, ids = route(...); y = experts(x2, ...)    (this library)
  h, x = combine_norm_sandwich(y, dense, ..., h, post_feedforward_layernorm, layer_scalar, next norm)
Several layers with their own weights run back to back in one graph; replays on new inputs, written
between replays by eager work, must give the bits of an eager run on the same inputs.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
H, E, K, I, ID = 2816, 128, 8, 704, 2112   # ID: the dense MLP's width, any value serves here
EPS = 1e-6


def _layers(n, fp8, seed):
    from flide_amd.kernels import moe

    g = torch.Generator(device=DEV).manual_seed(seed)
    bf = torch.bfloat16

    def rnd(*shape, s=0.02):
        return (torch.randn(*shape, generator=g, device=DEV) * s).to(bf)

    def norm_w():
        return (torch.rand(H, generator=g, device=DEV) + 0.5).to(bf)

    layers = []
    for _ in range(n):
        w = {"experts": rnd(E, 2 * I, H), "experts_down": rnd(E, H, I), "inter": I, "topk": K}
        if fp8:
            w["experts"], w["experts_scale"] = moe.quantize_experts(w["experts"])
            w["experts_down"], w["experts_down_scale"] = moe.quantize_experts(w["experts_down"])
        layers.append({
            "moe": w,
            "o_t": rnd(H, H).t().contiguous(),            # stand-in for attention's output product
            "gate_up_t": rnd(2 * ID, H).t().contiguous(),  # dense MLP, stored [in, out]
            "down_t": rnd(H, ID).t().contiguous(),
            "router": rnd(E, H),
            "router_norm": (torch.rand(H, generator=g, device=DEV) * 0.1).to(bf),
            "scale": (torch.rand(E, generator=g, device=DEV) + 0.5).to(bf),
            "post_attn": norm_w(), "pre_ffn": norm_w(), "pre_ffn_2": norm_w(),
            "post_ffn_1": norm_w(), "post_ffn_2": norm_w(), "post_ffn": norm_w(), "input": norm_w(),
            "scalar": torch.tensor([0.9], dtype=bf, device=DEV),
        })
    return layers


def _stack(layers, h_in):
    from flide_amd.kernels import moe
    from flide_amd.kernels import pointwise as pw

    def act(gu, n):
        return pw.geglu(gu[:, :n], gu[:, n:])

    h = h_in
    x = pw.rms_norm(h, layers[0]["input"], EPS, offset=False)
    for i, w in enumerate(layers):
        d = torch.mm(x, w["o_t"])
        df = d.float()
        d_n = (df * torch.rsqrt(df.pow(2).mean(-1, keepdim=True) + EPS)).to(torch.bfloat16) * w["post_attn"]
        h = (h.float() + d_n.float()).to(torch.bfloat16)
        x = pw.rms_norm(h, w["pre_ffn"], EPS, offset=False)
        gu = torch.mm(x, w["gate_up_t"])
        dense = torch.mm(pw.geglu(gu[:, :ID], gu[:, ID:]), w["down_t"])
        logits, x2 = moe.router_norm(h, w["router_norm"], w["router"], EPS, w["pre_ffn_2"])
        top, ids = moe.route(logits, K, w["scale"])
        y = moe.experts(x2, w["moe"], top, ids, act)
        nxt = layers[i + 1]["input"] if i + 1 < len(layers) else None
        h, x = moe.combine_norm_sandwich(y, dense, w["post_ffn_1"], w["post_ffn_2"], K, EPS, h, w["post_ffn"],
                                         w["scalar"], nxt)
    return h


@pytest.mark.parametrize("T,fp8", [(64, False), (1024, False), (64, True), (1024, True)])
def test_decoder_stack_capture(T, fp8):
    print(f"decoder stack capture T={T} fp8={fp8}", flush=True)
    n_layers = 4
    layers = _layers(n_layers, fp8, seed=7 + T + int(fp8))
    h_in = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(11)

    def new_input():
        h_in.copy_(torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16))

    new_input()
    _stack(layers, h_in)   # eager first: the activation callable is recognised outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _stack(layers, h_in)
    for rep in range(3):
        new_input()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = _stack(layers, h_in)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"replay {rep}: {(got != ref).sum().item()} elements differ"
    del graph, layers
    torch.cuda.empty_cache()
