"""Key maps and MoE layer loading from the reference's checkpoint formats (CPU, no kernels).

The key maps restate simple_inference_engine.py:139-145 (release -> native)
and conversion/convert_to_hf.py:17-30 (native -> release); the checks below
use the key shapes those files handle.  A synthetic release directory (two MoE
layers among unrelated tensors, written with safetensors) must load into
SparseMoESwiGLU layers with exactly its tensors, and save back to the same keys.
"""
import json

import pytest
import torch

from hrm_moe_amd import checkpoint as ck


def test_key_maps_follow_the_reference():
    assert ck.hf_to_native_key("model.H_module.layers.3.mlp.gate.weight") == "model.H_level.core.layers.3.mlp.gate.weight"
    assert ck.hf_to_native_key("model.L_module.layers.0.mlp.experts.down_weight") == \
        "model.L_level.core.layers.0.mlp.experts.down_weight"
    assert ck.hf_to_native_key("model.z_L_init") == "model.zL_init"
    assert ck.hf_to_native_key("model.embed_tokens.weight") == "embed_tokens.embedding_weight"
    assert ck.hf_to_native_key("lm_head.weight") == "lm_head.weight"
    assert ck.native_to_hf_key("model.zH_init") is None
    assert ck.native_to_hf_key("model.H_level.core.rotary_emb.cos_cached") is None
    for key in ("model.H_level.core.layers.7.mlp.experts.gate_up_weight", "model.zL_init",
                "embed_tokens.embedding_weight", "model.L_level.core.layers.1.self_attn.qkv_proj.weight"):
        assert ck.hf_to_native_key(ck.native_to_hf_key(key)) == key


def _release_dir(tmp_path, e=8, h=64, i=32, k=2):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    state = {"model.embed_tokens.weight": torch.randn(100, h, generator=g),
             "model.z_L_init": torch.randn(h, generator=g)}
    for prefix in ("model.H_module.layers.0.", "model.L_module.layers.1."):
        state[prefix + "self_attn.qkv_proj.weight"] = torch.randn(3 * h, h, generator=g)
        state[prefix + "mlp.gate.weight"] = torch.randn(e, h, generator=g)
        state[prefix + "mlp.experts.gate_up_weight"] = torch.randn(e, 2 * i, h, generator=g)
        state[prefix + "mlp.experts.down_weight"] = torch.randn(e, h, i, generator=g)
    save_file({k_: v.to(torch.bfloat16) for k_, v in state.items()}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"moe_num_experts": e, "moe_top_k": k,
                                                      "moe_norm_topk_prob": True}))
    return state


def test_load_and_save_round_trip(tmp_path):
    state = _release_dir(tmp_path)
    layers = ck.load_moe_layers(str(tmp_path), device="cpu", dtype=torch.bfloat16)
    assert sorted(layers) == ["model.H_level.core.layers.0.mlp.", "model.L_level.core.layers.1.mlp."]
    for prefix, layer in layers.items():
        assert (layer.num_experts, layer.top_k, layer.norm_topk_prob) == (8, 2, True)
        hf_prefix = ck.native_to_hf_key(prefix)
        for name in ck.MOE_PARAMS:
            assert torch.equal(layer.state_dict()[name], state[hf_prefix + name].to(torch.bfloat16)), name
    out = tmp_path / "moe_only.safetensors"
    ck.save_moe_layers(layers, str(out))
    from safetensors.torch import load_file
    saved = load_file(str(out))
    assert set(saved) == {p + n for p in ("model.H_module.layers.0.mlp.", "model.L_module.layers.1.mlp.")
                          for n in ck.MOE_PARAMS}
    for key, value in saved.items():
        assert torch.equal(value, state[key].to(torch.bfloat16))


def test_bad_shapes_and_missing_files(tmp_path):
    with pytest.raises(FileNotFoundError):
        ck.load_moe_layers(str(tmp_path), device="cpu")
    state = {"a.mlp.gate.weight": torch.zeros(4, 16), "a.mlp.experts.gate_up_weight": torch.zeros(4, 8, 16),
             "a.mlp.experts.down_weight": torch.zeros(4, 16, 5)}
    with pytest.raises(ValueError):
        ck.moe_layer_config(state, "a.mlp.")
    state["a.mlp.experts.down_weight"] = torch.zeros(4, 16, 4)
    assert ck.moe_layer_config(state, "a.mlp.") == dict(hidden_size=16, intermediate_size=4, num_experts=4, top_k=1,
                                                         norm_topk_prob=True)


@pytest.mark.gpu
def test_loaded_layer_runs_on_the_gpu(tmp_path, cuda):
    """A layer loaded from a release directory gives the oracle's output for the file's tensors."""
    import torch.nn.functional as F
    from safetensors.torch import save_file

    from hrm_moe_amd import ops
    from oracle import moe_oracle as mo
    from oracle import synth
    t, h, e, i, k = 256, 256, 8, 128, 2
    x, wg, wgu, wdn = synth.moe_inputs(31, t, h, e, i)
    bf = torch.bfloat16
    prefix = "model.H_module.layers.2.mlp."
    save_file({prefix + "gate.weight": torch.from_numpy(wg).to(bf),
               prefix + "experts.gate_up_weight": torch.from_numpy(wgu).to(bf),
               prefix + "experts.down_weight": torch.from_numpy(wdn).to(bf)}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"moe_top_k": k, "moe_norm_topk_prob": True}))
    layer = ck.load_moe_layers(str(tmp_path), device=cuda)["model.H_level.core.layers.2.mlp."]
    xb = torch.from_numpy(x).to(bf)
    with torch.no_grad():
        out = layer(xb.to(cuda))
        logits = F.linear(xb.to(cuda), layer.gate.weight)
        idx = ops.router_topk(logits, k, True, bf)[2]
    ref, im = mo.moe_forward(xb, *(torch.from_numpy(a).to(bf) for a in (wg, wgu, wdn)), k, True,
                             intermediates=True, logits=logits.cpu())
    assert torch.equal(idx.cpu(), im["idx"])
    rel = (out.float().cpu() - ref.float()).abs().max().item() / ref.float().abs().max().item()
    assert rel <= 2e-2
