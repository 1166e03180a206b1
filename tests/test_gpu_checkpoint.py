"""The checkpoint loader on the GPU: a checkpoint in the reference's format (tensor names, FP8 [N, K]
with BF16 [N, 1] scales, NVFP4 U8 [N, K/2] with E4M3 [N, K/16] block scales and an F32 global
scale g; FO/src/host/load.rs) is written with the `safetensors` package for one sliding layer
(index 4) and one full-attention layer (index 5) at their real shapes. load_model reads it into
device tensors, which must hold the file's bytes (the global scales as 1 / g, the layer scalar
eight times), and the operators must give the oracle's results when they take their weights from
the loaded tensors."""
import numpy as np
import pytest

from gpu_util import dev, gate, host, need_gpu, say, torch
from kat_inputs import unbf
from moa_amd import prng, synth
from oracle import oracle as O
from test_gpu_ffn import FFN_ATOL, oracle_nvfp4

pytestmark = pytest.mark.gpu
H, L = 3840, 15360


def _fp8(rng, rows, cols):
    c = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    return np.where((c & 0x7F) == 0x7F, c ^ 1, c).astype(np.uint8)  # no NaN codes


def _bf16(x):
    return prng.f32_to_bf16_bits(np.asarray(x, np.float32))


def make_checkpoint(path):
    """Tensors of layers 4 (sliding) and 5 (full) plus the final norm, by load.rs's names, and the
    host copies the checks compare against."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(0)
    ref = synth.ref_ffn_inputs(0)  # the reference harness's NVFP4 MLP (codes, E4M3 scales, 1 / g)
    host_t = {}

    def put(name, arr, dtype):
        host_t[name] = (np.ascontiguousarray(arr), dtype)

    put("model.language_model.norm.weight", _bf16(1.0 + 0.1 * rng.standard_normal(H)), "bf16")
    for layer, full in ((4, False), (5, True)):
        p = f"model.language_model.layers.{layer}"
        a = f"{p}.self_attn"
        q_rows, k_rows, d = (8192, 512, 512) if full else (4096, 2048, 256)
        projs = [("q_proj", q_rows), ("k_proj", k_rows)] + ([] if full else [("v_proj", k_rows)])
        for name, rows in projs:
            put(f"{a}.{name}.weight", _fp8(rng, rows, H), "f8")
            put(f"{a}.{name}.weight_scale", _bf16(1e-3 * (0.5 + rng.random((rows, 1)))), "bf16")
        put(f"{a}.o_proj.weight", _fp8(rng, H, q_rows), "f8")
        put(f"{a}.o_proj.weight_scale", _bf16(1e-3 * (0.5 + rng.random((H, 1)))), "bf16")
        put(f"{a}.q_norm.weight", _bf16(1.0 + 0.1 * rng.standard_normal(d)), "bf16")
        put(f"{a}.k_norm.weight", _bf16(1.0 + 0.1 * rng.standard_normal(d)), "bf16")
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm"):
            put(f"{p}.{n}.weight", _bf16(0.75 + 0.5 * rng.random(H)), "bf16")
        put(f"{p}.layer_scalar", _bf16([0.375]), "bf16")
        for n in ("up", "gate", "down"):
            m = f"{p}.mlp.{n}_proj"
            # layer 5 stores the same codes rotated by one byte, so a mix-up of layers shows
            put(f"{m}.weight_packed", np.roll(ref[f"{n}_weight_packed"], layer - 4), "u8")
            put(f"{m}.weight_scale", np.roll(ref[f"{n}_weight_scale"], layer - 4), "f8")
            put(f"{m}.weight_global_scale", np.float32(1.0) / ref[f"{n}_global_scale"] * np.float32(layer - 3), "f32")
    conv = {"bf16": lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16),
            "f8": lambda a: torch.from_numpy(a).view(torch.float8_e4m3fn),
            "u8": lambda a: torch.from_numpy(a), "f32": lambda a: torch.from_numpy(a)}
    save_file({k: conv[dt](a) for k, (a, dt) in host_t.items()}, str(path))
    return {k: a for k, (a, _) in host_t.items()}, ref


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    need_gpu()
    from moa_amd import checkpoint
    path = tmp_path_factory.mktemp("ckpt") / "model.safetensors"
    say("checkpoint: writing layers 4 and 5 at real shapes")
    src, ref = make_checkpoint(path)
    say(f"checkpoint: {path.stat().st_size / 2**20:.0f} MiB written, loading")
    model = checkpoint.load_model(path, layers=[4, 5], embedding=False)
    torch.cuda.synchronize()
    return model, src, ref


def _bytes(t):
    return t.contiguous().view(torch.uint8).cpu().numpy().reshape(-1)


def test_device_tensors_hold_the_file_bytes(loaded):
    model, src, _ = loaded
    from moa_amd import checkpoint
    assert isinstance(model.layers[4], checkpoint.SlidingLayer)
    assert isinstance(model.layers[5], checkpoint.FullLayer)
    assert np.array_equal(_bytes(model.final_norm), src["model.language_model.norm.weight"].view(np.uint8))
    names = {"input_norm": "input_layernorm.weight", "post_attention_norm": "post_attention_layernorm.weight",
             "pre_feedforward_norm": "pre_feedforward_layernorm.weight",
             "post_feedforward_norm": "post_feedforward_layernorm.weight", "q_weight": "self_attn.q_proj.weight",
             "k_weight": "self_attn.k_proj.weight", "v_weight": "self_attn.v_proj.weight",
             "q_weight_scale": "self_attn.q_proj.weight_scale", "k_weight_scale": "self_attn.k_proj.weight_scale",
             "v_weight_scale": "self_attn.v_proj.weight_scale", "q_norm": "self_attn.q_norm.weight",
             "k_norm": "self_attn.k_norm.weight", "o_weight": "self_attn.o_proj.weight",
             "o_weight_scale": "self_attn.o_proj.weight_scale"}
    checked = 0
    for i, layer in model.layers.items():
        for field, name in names.items():
            if not hasattr(layer, field):
                continue
            want = src[f"model.language_model.layers.{i}.{name}"]
            assert np.array_equal(_bytes(getattr(layer, field)), want.reshape(-1).view(np.uint8)), (i, field)
            checked += 1
        m = f"model.language_model.layers.{i}.mlp"
        for n in ("up", "gate", "down"):
            assert np.array_equal(_bytes(getattr(layer.mlp, f"{n}_weight_packed")),
                                  src[f"{m}.{n}_proj.weight_packed"].reshape(-1)), (i, n)
            assert np.array_equal(_bytes(getattr(layer.mlp, f"{n}_weight_scale")),
                                  src[f"{m}.{n}_proj.weight_scale"].reshape(-1)), (i, n)
            g = src[f"{m}.{n}_proj.weight_global_scale"][0]
            assert getattr(layer.mlp, f"{n}_global_scale").item() == np.float32(1.0) / g, (i, n)
        ls = _bytes(layer.layer_scalar).view(np.uint16)
        assert ls.size == 8 and np.all(ls == src[f"model.language_model.layers.{i}.layer_scalar"][0])
    assert checked == 14 + 12


def test_operators_run_on_the_loaded_weights(loaded):
    model, src, ref = loaded
    from moa_amd import ops
    L4 = model.layers[4]
    rng = np.random.default_rng(1)
    # O projection (FP8 + BF16 column scales) of layer 4
    x = _bf16(rng.standard_normal(4096))
    res = _bf16(rng.standard_normal(H))
    r = dev(res)
    ops.sliding_attention_output(dev(x), L4.post_attention_norm, L4.o_weight, L4.o_weight_scale, r)
    a = "model.language_model.layers.4"
    want = res.copy()
    O.sliding_attention_output(x, src[f"{a}.post_attention_layernorm.weight"], src[f"{a}.self_attn.o_proj.weight"],
                               unbf(src[f"{a}.self_attn.o_proj.weight_scale"].reshape(-1)), want)
    gate(want, host(r), "o on loaded layer 4")
    # NVFP4 FFN of layer 4 (E2M1 + E4M3 block scales + 1 / g from the file)
    d = dict(residual=_bf16(rng.standard_normal(H)), pre_ff_rms_weight=src[f"{a}.pre_feedforward_layernorm.weight"],
             post_ff_rms_weight=src[f"{a}.post_feedforward_layernorm.weight"],
             layer_scalar=np.repeat(src[f"{a}.layer_scalar"], 8))
    for n in ("up", "gate", "down"):
        d[f"{n}_weight_packed"] = ref[f"{n}_weight_packed"]
        d[f"{n}_weight_scale"] = ref[f"{n}_weight_scale"]
        d[f"{n}_global_scale"] = np.array([getattr(L4.mlp, f"{n}_global_scale").item()], np.float32)
    r = dev(d["residual"])
    m = L4.mlp
    ops.decoder_feedforward(r, L4.pre_feedforward_norm, m.up_weight_packed, m.gate_weight_packed, m.down_weight_packed,
                            m.up_weight_scale, m.gate_weight_scale, m.down_weight_scale, m.up_global_scale,
                            m.gate_global_scale, m.down_global_scale, L4.post_feedforward_norm, L4.layer_scalar)
    gate(oracle_nvfp4(d), host(r), "nvfp4 ffn on loaded layer 4", atol=FFN_ATOL)
