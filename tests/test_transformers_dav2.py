"""The whole Depth Anything V2 Small against `transformers`' own implementation
(DepthAnythingForDepthEstimation, the model the reference's Python script
and its real-weight tests compare with: tests/depth_anything_v2.rs:407-599,
scripts/reference/depth_anything_v2.py). No weights are fetched: the model is
built from its configuration and every parameter drawn at random, so every
term of the forward pass counts.

The state dict goes through a safetensors file into the loader (inventory
check, conversions, the position embedding resampled from 37 x 37 to the
test image's grid), then through the oracle's composition of the encoder and
decoder; features and depth must agree with transformers' float32 forward pass
within the reference's feature tolerance (max 2e-3, mean 5e-5:
load/depth_anything_v2/reference.rs:198-244). This pins the loader's name
and layout mapping, the position resampling and the decoder's wiring against
an implementation that is not the reference's. CPU only; the GPU path runs the
same comparison in tests/test_gpu_load.py.
"""

import numpy as np
import pytest
import torch

import oracle
from beatlm_amd import ir, load
from tests.test_gpu_dpt import oracle_encoder

transformers = pytest.importorskip("transformers")

MAX_ERR, MEAN_ERR = 2e-3, 5e-5


def hf_model(seed=0):
    from transformers import DepthAnythingConfig, DepthAnythingForDepthEstimation, Dinov2Config

    backbone = Dinov2Config(image_size=518, patch_size=14, num_channels=3, hidden_size=384, num_hidden_layers=12,
                            num_attention_heads=6, mlp_ratio=4, out_indices=[3, 6, 9, 12], apply_layernorm=True,
                            reshape_hidden_states=False, layerscale_value=1.0)
    config = DepthAnythingConfig(backbone_config=backbone, reassemble_hidden_size=384, patch_size=14,
                                 reassemble_factors=[4, 2, 1, 0.5], neck_hidden_sizes=[48, 96, 192, 384],
                                 fusion_hidden_size=64, head_in_index=-1, head_hidden_size=32,
                                 depth_estimation_type="relative", max_depth=None)
    torch.manual_seed(seed)
    model = DepthAnythingForDepthEstimation(config).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name and name.endswith("weight"):
                v = torch.rand(p.shape, generator=g) * 0.4 + 0.8
            elif "lambda1" in name:
                v = torch.rand(p.shape, generator=g) * 0.9 + 0.1
            elif name.endswith("bias"):
                v = (torch.rand(p.shape, generator=g) - 0.5) * 0.2
            elif p.dim() >= 2 and not name.endswith(("cls_token", "mask_token", "position_embeddings")):
                # fan-in: a transposed convolution's is its input channels
                fan = p.shape[0] if "neck.reassemble_stage" in name and "resize" in name and p.shape[2] != 3 \
                    else int(np.prod(p.shape[1:]))
                v = (torch.rand(p.shape, generator=g) * 2 - 1) / np.sqrt(fan)
            else:
                v = (torch.rand(p.shape, generator=g) - 0.5)
            p.copy_(v)
    return model


@pytest.fixture(scope="module")
def model_and_file():
    from safetensors.torch import save

    model = hf_model()
    return model, save({k: v.contiguous() for k, v in model.state_dict().items()})


def test_the_inventory_is_exactly_transformers_state_dict(model_and_file):
    _, data = model_and_file
    report = load.inventory(ir.DepthConfig.small()).check(load.Archive.parse(data))
    assert report.is_exact(), str(report)
    assert report.file_parameters == 24_785_089


@pytest.mark.parametrize("side", [98, 70])
def test_features_and_depth_match_transformers(model_and_file, side):
    model, data = model_and_file
    cfg = ir.DepthConfig.small()
    grid = side // cfg.patch_size
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    numbers = load.depth_weights(load.Archive.parse(data), cfg, m, side)

    rng = np.random.default_rng(side)
    mean = np.array([0.485, 0.456, 0.406], np.float32)
    std = np.array([0.229, 0.224, 0.225], np.float32)
    image = ((rng.uniform(0, 1, (side, side, 3)).astype(np.float32) - mean) / std).astype(np.float32)
    values = dict(numbers)
    values[m.encoder.embed.image] = image.ravel()

    features = oracle_encoder(m.encoder, cfg, grid, values)
    named = {name: numbers[tid] for tid, name, _ in m.decoder_weights}
    depth = oracle.depth_decoder(cfg, side, features, named)

    with torch.no_grad():
        pixels = torch.from_numpy(image).permute(2, 0, 1)[None]
        maps = model.backbone(pixels).feature_maps
        want_depth = model(pixel_values=pixels).predicted_depth[0].numpy()
    for tap, (got, hf) in enumerate(zip(features, maps)):
        want = hf[0, 1:].numpy().ravel()  # the class token dropped, as the neck's readout does
        err = np.abs(got - want)
        assert err.max() <= MAX_ERR and err.mean() <= MEAN_ERR, (tap, err.max(), err.mean())
    # The depth of random weights is small (here about 0.03 at most): the
    # tolerance scales with its largest value, and a quarter of it at least
    # must be positive after the final ReLU for the comparison to mean much.
    want_depth = want_depth.ravel()
    err = np.abs(depth - want_depth)
    scale = float(np.abs(want_depth).max())
    assert scale > 0 and (want_depth > 0).mean() > 0.1
    assert err.max() <= MAX_ERR * scale and err.mean() <= MEAN_ERR * scale, (err.max(), err.mean(), scale)
