"""INT8 checkpoint layout: plan, rank slicing, validation (CPU), and a
loaded block's FFN against the oracle (GPU)."""
import json

import numpy as np
import pytest
import torch

from w8a8 import checkpoint as ck


def _dit_weights(g, hidden=512, ffn=1024):
    def q(n, k):
        return torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8), torch.rand((n, 1), generator=g) * 1e-3
    weights = {'qkv_proj': q(3 * hidden, hidden), 'out_proj': q(hidden, hidden), 'fc1': q(2 * ffn, hidden),
               'fc2': q(hidden, ffn)}
    rep = {'norm1.weight': torch.rand(hidden, generator=g), 'norm2.weight': torch.rand(hidden, generator=g),
           'q_norm.weight': torch.rand(128, generator=g), 'k_norm.weight': torch.rand(128, generator=g),
           'adaln_proj.weight': torch.randn((18 * hidden, 8), generator=g),
           'adaln_proj.bias': torch.randn(18 * hidden, generator=g)}
    return weights, rep


@pytest.fixture
def dit_file(tmp_path):
    g = torch.Generator().manual_seed(0)
    weights, rep = _dit_weights(g)
    path = ck.save_block(tmp_path / 'dit.safetensors', 'dit', 3, weights, rep)
    return path, weights, rep


def test_full_block_loads_exactly(dit_file):
    path, weights, rep = dit_file
    block = ck.load_block(path, 'dit', 3, device='cpu')
    for name, (w, s) in weights.items():
        m = getattr(block, name)
        assert torch.equal(m.weight.data, w) and torch.equal(m.weight_scale.data, s)
    for name, t in rep.items():
        assert torch.equal(block.tensor(name), t)
    assert block.fc1.components == 2 and block.qkv_proj.components == 3
    assert all(v == ck.QUANT_CONFIG for v in block._rank_checkpoint_metadata.values())


def test_rank_halves_are_component_wise_and_k_split(dit_file):
    path, weights, _ = dit_file
    r0 = ck.load_block(path, 'dit', 3, rank=0, world_size=2, device='cpu')
    r1 = ck.load_block(path, 'dit', 3, rank=1, world_size=2, device='cpu')
    w = weights['qkv_proj'][0]
    chunk = w.shape[0] // 3
    for i in range(3):   # component i: rank 0 takes its first half, rank 1 its second
        part0 = r0.qkv_proj.weight.data[i * chunk // 2:(i + 1) * chunk // 2]
        part1 = r1.qkv_proj.weight.data[i * chunk // 2:(i + 1) * chunk // 2]
        assert torch.equal(torch.cat([part0, part1]), w[i * chunk:(i + 1) * chunk])
    w2 = weights['fc2'][0]
    assert torch.equal(torch.cat([r0.fc2.weight.data, r1.fc2.weight.data], 1), w2)
    assert torch.equal(r0.fc2.weight_scale.data, weights['fc2'][1])   # row scales replicated
    assert r0.fc1.weight.shape == (1024, 512) and r1.out_proj.weight.shape == (512, 256)


def test_plan_rejects_unqualified_layouts(tmp_path):
    g = torch.Generator().manual_seed(1)
    weights, rep = _dit_weights(g, hidden=512, ffn=768)
    path = ck.save_block(tmp_path / 'a.safetensors', 'dit', 0, weights, rep)
    with pytest.raises(ValueError, match='ConvRot groups'):   # fc2 K = 768 splits into 384-channel halves
        ck.load_block(path, 'dit', 0, rank=0, world_size=2, device='cpu')
    ck.load_block(path, 'dit', 0, device='cpu')                # whole rows are fine on one GPU
    from safetensors.torch import load_file, save_file
    state = load_file(str(path))
    bad = dict(state)
    bad['blocks.0.mlp.fc1.weight'] = bad['blocks.0.mlp.fc1.weight'].to(torch.float16)
    save_file(bad, str(tmp_path / 'b.safetensors'))
    with pytest.raises(ValueError, match='dtype'):
        ck.load_block(tmp_path / 'b.safetensors', 'dit', 0, device='cpu')
    extra = dict(state)
    extra['blocks.0.mlp.fc3.weight'] = torch.zeros(2, 2)
    save_file(extra, str(tmp_path / 'c.safetensors'))
    with pytest.raises(ValueError, match='Unqualified'):
        ck.load_block(tmp_path / 'c.safetensors', 'dit', 0, device='cpu')
    meta = dict(state)
    meta['blocks.0.attn.qkv_proj.comfy_quant'] = torch.tensor(list(json.dumps(
        {'format': 'int8_tensorwise', 'convrot': False, 'convrot_groupsize': 256}).encode()), dtype=torch.uint8)
    save_file(meta, str(tmp_path / 'd.safetensors'))
    with pytest.raises(ValueError, match='metadata'):
        ck.load_block(tmp_path / 'd.safetensors', 'dit', 0, device='cpu')
    missing = {k: v for k, v in state.items() if 'out_proj.weight_scale' not in k}
    save_file(missing, str(tmp_path / 'e.safetensors'))
    with pytest.raises(ValueError, match='Missing'):
        ck.load_block(tmp_path / 'e.safetensors', 'dit', 0, device='cpu')
    with pytest.raises(ValueError):
        ck.load_block(path, 'vae', 0, device='cpu')


def test_te_block_layout(tmp_path):
    g = torch.Generator().manual_seed(2)
    def q(n, k):
        return torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8), torch.rand((n, 1), generator=g)
    h, f = 512, 1024
    weights = {'q_proj': q(h, h), 'k_proj': q(h // 2, h), 'v_proj': q(h // 2, h), 'o_proj': q(h, h),
               'gate_proj': q(f, h), 'up_proj': q(f, h), 'down_proj': q(h, f)}
    rep = {'input_layernorm.weight': torch.rand(h, generator=g), 'q_norm.weight': torch.rand(128, generator=g),
           'post_attention_layernorm.weight': torch.rand(h, generator=g), 'k_norm.weight': torch.rand(128, generator=g)}
    path = ck.save_block(tmp_path / 'te.safetensors', 'te', 7, weights, rep)
    b = ck.load_block(path, 'te', 7, rank=1, world_size=2, device='cpu')
    assert torch.equal(b.k_proj.weight.data, weights['k_proj'][0][h // 4:])
    assert torch.equal(b.down_proj.weight.data, weights['down_proj'][0][:, f // 2:])
    # replicated TE tensors take the FP16 of the reference's TE module shells
    assert b.tensor('q_norm.weight').dtype == torch.float16
    assert torch.equal(b.tensor('q_norm.weight'), rep['q_norm.weight'].half())
    partial = {k: v for k, v in rep.items() if k != 'post_attention_layernorm.weight'}
    ck.save_block(tmp_path / 'te2.safetensors', 'te', 7, weights, partial)
    with pytest.raises(ValueError, match='Missing replicated'):
        ck.load_block(tmp_path / 'te2.safetensors', 'te', 7, device='cpu')
    bad = dict(weights, down_proj=q(h, f // 2))
    ck.save_block(tmp_path / 'te3.safetensors', 'te', 7, bad, rep)
    with pytest.raises(ValueError, match='shape differs'):
        ck.load_block(tmp_path / 'te3.safetensors', 'te', 7, device='cpu')


def test_dit_replicated_tensors_required_and_checked(tmp_path):
    g = torch.Generator().manual_seed(4)
    weights, rep = _dit_weights(g)
    for drop in ('norm1.weight', 'adaln_proj.bias'):
        ck.save_block(tmp_path / 'm.safetensors', 'dit', 0, weights, {k: v for k, v in rep.items() if k != drop})
        with pytest.raises(ValueError, match='Missing replicated'):
            ck.load_block(tmp_path / 'm.safetensors', 'dit', 0, device='cpu')
    for key, bad in (('norm2.weight', torch.rand(256)), ('k_norm.weight', torch.rand(64)),
                     ('adaln_proj.weight', torch.rand(6 * 512, 8))):
        ck.save_block(tmp_path / 's.safetensors', 'dit', 0, weights, dict(rep, **{key: bad}))
        with pytest.raises(ValueError, match='shape differs'):
            ck.load_block(tmp_path / 's.safetensors', 'dit', 0, device='cpu')
    w = dict(weights, fc2=(weights['fc2'][0][:, :512].contiguous(), weights['fc2'][1]))
    ck.save_block(tmp_path / 'f.safetensors', 'dit', 0, w, rep)
    with pytest.raises(ValueError, match='shape differs'):
        ck.load_block(tmp_path / 'f.safetensors', 'dit', 0, device='cpu')
    # FP16 replicated tensors in the file load as the DiT shells' FP32
    half = {k: v.half() for k, v in rep.items()}
    ck.save_block(tmp_path / 'h.safetensors', 'dit', 0, weights, half)
    b = ck.load_block(tmp_path / 'h.safetensors', 'dit', 0, device='cpu')
    assert b.tensor('norm1.weight').dtype == torch.float32
    assert torch.equal(b.tensor('norm1.weight'), half['norm1.weight'].float())


@pytest.mark.gpu
def test_loaded_block_ffn_matches_oracle(gpu, dit_file):
    import oracle as o
    from helpers import assert_bits_equal, np_of
    from w8a8 import tp_dit
    path, weights, _ = dit_file
    block = ck.load_block(path, 'dit', 3, device=gpu)
    ffn = tp_dit.DiTFeedForwardINT8.from_projections(block.fc1, block.fc2)
    g = torch.Generator().manual_seed(9)
    h = torch.randn((77, 512), generator=g).half()
    res = (torch.randn((77, 512), generator=g) / 512).half()
    out = ffn(h.to(gpu), res.to(gpu))
    want = o.ffn_block(np_of(h), np_of(weights['fc1'][0]), np_of(weights['fc1'][1]).reshape(-1),
                       np_of(weights['fc2'][0]), np_of(weights['fc2'][1]).reshape(-1), np_of(res))
    assert_bits_equal(np_of(out), want, 'ffn from a loaded checkpoint')
