"""Compiled DiT blocks on the FP8 path: no graph breaks, same results as eager.

The reference compiles every DiT block with torch.compile (runtime/model_manager.py:127-141,
COMPILE_MODE config.py:30) while the FP8 linears and the routed SDPA run inside them.  Each
launch here is a torch.library custom op with a fake kernel, so the traced block must stay
one graph with the FP8 kernels as nodes.  Dynamo is run with the "eager" backend (the graph
is executed by torch, no code generation).
"""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

C, H, D = 256, 2, 128


class GELUProj(nn.Module):
    def __init__(self, a, b):
        super().__init__()
        self.proj = nn.Linear(a, b)
        self.approximate = "tanh"

    def forward(self, x):
        return F.gelu(self.proj(x), approximate=self.approximate)


class Block(nn.Module):
    """adaLN -> QKV -> routed SDPA -> out, adaLN -> MLP (tanh-GELU) -> down, with residuals."""

    def __init__(self, fused_adaln):
        super().__init__()
        self.fused_adaln = fused_adaln
        self.qkv, self.out = nn.Linear(C, 3 * C), nn.Linear(C, C)
        self.up, self.down = GELUProj(C, 4 * C), nn.Linear(4 * C, C)

    def forward(self, x, shift, scale):
        from minimaxh3_amd.kernels import fp8_linear as fl
        B, S, _ = x.shape
        if self.fused_adaln:
            x8, sa = fl.adaln_quantize_rows(x, shift, scale)
            qkv = self.qkv.forward_quantized(x8, sa).view(B, S, 3, H, D)
        else:
            h = F.layer_norm(x, (C,), eps=1e-6) * (1 + scale[:, None]) + shift[:, None]
            qkv = self.qkv(h).view(B, S, 3, H, D)
        q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
        a = F.scaled_dot_product_attention(q, k, v).permute(0, 2, 1, 3).reshape(B, S, C)
        x = x + self.out(a)
        h2 = F.layer_norm(x, (C,), eps=1e-6) * (1 + scale[:, None]) + shift[:, None]
        return x + self.down(self.up(h2))


class Model(nn.Module):
    def __init__(self, fused_adaln):
        super().__init__()
        self.blocks = nn.ModuleList([Block(fused_adaln) for _ in range(3)])


@pytest.mark.gpu
@pytest.mark.parametrize("fused_adaln", [False, True])
def test_compiled_block_one_graph_same_result(fused_adaln):
    import torch._dynamo as dynamo
    from minimaxh3_amd.kernels import attention_router as ar
    from minimaxh3_amd.kernels import fp8_linear as fl
    print(f"[compile] fused_adaln={fused_adaln}", flush=True)
    saved = (ar.enabled, ar.repair_tau, ar.min_seq)
    saved_sdpa = (F.scaled_dot_product_attention, getattr(torch._C._nn, "scaled_dot_product_attention", None),
                  ar._installed)
    ar.install()
    ar.configure(True, -1.0, 128)
    try:
        torch.manual_seed(0)
        m = Model(fused_adaln).cuda().to(torch.bfloat16)
        assert fl.convert_transformer_to_fp8(m, "", 0, fuse_gelu=True) == 3 * 4
        blk = m.blocks[1]
        x = torch.randn(1, 300, C, device="cuda").to(torch.bfloat16)
        shift = (torch.randn(1, C, device="cuda") * 0.1).to(torch.bfloat16)
        scale = (torch.randn(1, C, device="cuda") * 0.1).to(torch.bfloat16)
        with ar.denoiser_scope(), torch.no_grad():
            ref = blk(x, shift, scale)
            dynamo.reset()
            ex = dynamo.explain(blk)(x, shift, scale)
            assert ex.graph_break_count == 0 and ex.graph_count == 1, [str(r.reason) for r in ex.break_reasons]
            targets = {str(n.target) for g in ex.graphs for n in g.graph.nodes}
            # q is a view of the fused projection output, so the Q quantizer runs inside
            # the attention launch (mxf8.attn_fwd_q)
            for op in ("mxf8.gemm_rowwise", "mxf8.attn_fwd_q", "mxf8.attn_quant_kv"):
                assert any(op in t for t in targets), (op, sorted(targets))
            if fused_adaln:
                assert any("mxf8.adaln_quant_rows" in t for t in targets)
            dynamo.reset()
            out = torch.compile(blk, backend="eager", fullgraph=True, dynamic=False)(x, shift, scale)
        assert torch.equal(out, ref)
    finally:
        ar.configure(*saved)
        F.scaled_dot_product_attention = saved_sdpa[0]
        if saved_sdpa[1] is not None:
            torch._C._nn.scaled_dot_product_attention = saved_sdpa[1]
        ar._installed = saved_sdpa[2]
        torch._dynamo.reset()


def _fp8_modules(blk):
    from minimaxh3_amd.kernels import fp8_linear as fl
    return [m for m in blk.modules() if isinstance(m, fl.FP8Linear)]


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["counting", "inductor"])
def test_lora_appended_after_compile(backend):
    """The reference compiles each block first (runtime/model_manager.py:127-141, dynamic=False,
    fullgraph=False) and only then does LoraManager.activate append (A, B, scale) to every
    targeted FP8Linear's adapters (runtime/lora.py:263-302); deactivate clears them again
    (303-309).  The compiled block must trace the adapter state without graph breaks, compile
    at most once more for it, and give the eager block's output (bit for bit with a backend
    that runs the traced graph as is; within the GEMM bar under Inductor, whose fused
    pointwise code rounds the bf16 LayerNorm / modulation differently from eager)."""
    import torch._dynamo as dynamo
    from minimaxh3_amd.kernels import attention_router as ar
    from minimaxh3_amd.kernels import fp8_linear as fl
    print(f"[compile lora] backend={backend}", flush=True)
    saved = (ar.enabled, ar.repair_tau, ar.min_seq)
    saved_sdpa = (F.scaled_dot_product_attention, getattr(torch._C._nn, "scaled_dot_product_attention", None),
                  ar._installed)
    ar.install()
    ar.configure(True, -1.0, 128)
    try:
        torch.manual_seed(1)
        m = Model(False).cuda().to(torch.bfloat16)
        fl.convert_transformer_to_fp8(m, "", 0, fuse_gelu=True)
        blk = m.blocks[1]
        x = torch.randn(1, 300, C, device="cuda").to(torch.bfloat16)
        shift = (torch.randn(1, C, device="cuda") * 0.1).to(torch.bfloat16)
        scale = (torch.randn(1, C, device="cuda") * 0.1).to(torch.bfloat16)
        graphs = []

        def counting(gm, example_inputs):
            graphs.append(gm)
            return gm.forward

        dynamo.reset()
        if backend == "counting":
            cblk = torch.compile(blk, backend=counting, dynamic=False, fullgraph=False)
        else:
            cblk = torch.compile(blk, mode="max-autotune-no-cudagraphs", dynamic=False, fullgraph=False)

        def same(a, b):
            if backend == "counting":
                assert torch.equal(a, b)
            else:
                err = (a.float() - b.float()).abs().max().item()
                assert err <= 1e-2 * b.float().abs().max().item(), err

        adapters = {id(mod): ((torch.randn(64, mod.in_features, device="cuda") * 0.02).to(torch.bfloat16),
                              (torch.randn(mod.out_features, 64, device="cuda") * 0.02).to(torch.bfloat16))
                    for mod in _fp8_modules(blk)}
        assert len(adapters) == 4
        with ar.denoiser_scope(), torch.no_grad():
            ref0 = blk(x, shift, scale)
            same(cblk(x, shift, scale), ref0)
            n0 = len(graphs)
            # activate: the runtime appends the adapter tensors after compilation
            for mod in _fp8_modules(blk):
                a, b = adapters[id(mod)]
                mod.adapters.append((a, b, 1.0))
            ref1 = blk(x, shift, scale)
            assert not torch.equal(ref1, ref0)  # the adapters change the output
            same(cblk(x, shift, scale), ref1)
            same(cblk(x, shift, scale), ref1)
            n1 = len(graphs)
            # deactivate: back to the adapter-free state
            for mod in _fp8_modules(blk):
                mod.adapters.clear()
            same(cblk(x, shift, scale), ref0)
            n2 = len(graphs)
            if backend == "counting":
                assert n0 == 1 and n1 - n0 <= 1 and n2 == n1, (n0, n1, n2)
                # the adapter state traces as one graph (no breaks)
                for mod in _fp8_modules(blk):
                    a, b = adapters[id(mod)]
                    mod.adapters.append((a, b, 1.0))
                ex = dynamo.explain(blk)(x, shift, scale)
                assert ex.graph_break_count == 0 and ex.graph_count == 1, [str(r.reason) for r in ex.break_reasons]
                targets = {str(n.target) for g in ex.graphs for n in g.graph.nodes}
                assert any("mxf8.lora_down" in t for t in targets), sorted(targets)
                for mod in _fp8_modules(blk):
                    mod.adapters.clear()
    finally:
        ar.configure(*saved)
        F.scaled_dot_product_attention = saved_sdpa[0]
        if saved_sdpa[1] is not None:
            torch._C._nn.scaled_dot_product_attention = saved_sdpa[1]
        ar._installed = saved_sdpa[2]
        torch._dynamo.reset()
