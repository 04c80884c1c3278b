"""A checkpoint on disk through the loader to the GPU: a safetensors file of a
Depth Anything V2 configuration (the checkpoint's names, shapes and PyTorch
layouts, random numbers), opened with Archive.open, checked against the
inventory, converted by depth_weights for an image of another size than the
checkpoint's (the position embedding resampled from a 5 x 5 to a 7 x 7
grid), written into a depth-model graph and run; the depth must match the
oracle's composition of the same model on the same converted numbers
(f32: |got - want| <= 1e-4 + 1e-4 |want|). The conversions themselves are
pinned on the CPU (tests/test_load.py)."""

from dataclasses import replace

import numpy as np
import pytest
import safetensors.numpy as stn

import oracle
from beatlm_amd import ir, load
from tests.test_gpu_dpt import oracle_decoder, oracle_encoder

pytestmark = pytest.mark.gpu


def checkpoint(cfg, path, seed=5):
    """Random numbers of every tensor the inventory lists, scaled as a trained
    model's are (weights U(+-1/sqrt(fan_in)), norms near 1, LayerScale in
    [0.1, 1]), in the checkpoint's own layouts."""
    rng = np.random.default_rng(seed)
    out = {}
    for s in load.inventory(cfg):
        n, shape = s.name, s.shape
        if n.endswith("norm1.weight") or n.endswith("norm2.weight") or n == "backbone.layernorm.weight":
            v = rng.uniform(0.8, 1.2, shape)
        elif "lambda1" in n:
            v = rng.uniform(0.1, 1.0, shape)
        elif n.endswith(".bias"):
            v = rng.uniform(-0.1, 0.1, shape)
        elif "position_embeddings" in n:
            v = rng.uniform(-0.5, 0.5, shape)
        elif "cls_token" in n or "mask_token" in n:
            v = rng.uniform(-1.0, 1.0, shape)
        else:
            # [out][in] or [out][in][kh][kw], except a transposed convolution's
            # [in][out][kh][kw]: fan-in is the product of all but the first
            # (for the transposed convolution, its input channels).
            fan = int(np.prod(shape[1:])) if not (".resize." in n and shape[2] != 3) else shape[0]
            v = rng.uniform(-1.0, 1.0, shape) / np.sqrt(fan)
        out[n] = np.asarray(v, np.float32)
    stn.save_file(out, str(path))


def test_a_checkpoint_file_runs_through_the_loader_on_the_gpu(ctx, tmp_path):
    cfg = replace(ir.DepthConfig.small(), image_size=70, num_layers=4, out_indices=(1, 2, 3, 4))
    path = tmp_path / "dav2.safetensors"
    checkpoint(cfg, path)
    archive = load.Archive.open(path)
    assert load.inventory(cfg).check(archive).is_exact()

    side = 98  # a 7 x 7 grid from the checkpoint's 5 x 5
    grid = side // cfg.patch_size
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    numbers = load.depth_weights(archive, cfg, m, side)
    image = oracle.uniform(77, side * side * 3, 0.0, 1.0)
    values = dict(numbers)
    values[m.encoder.embed.image] = image

    named = {name: numbers[tid] for tid, name, _ in m.decoder_weights}
    features = oracle_encoder(m.encoder, cfg, grid, values)
    want = oracle_decoder(cfg, side, features, named)
    got = ir.run_on_gpu(ctx, g, values)[m.depth]
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"depth element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"


@pytest.mark.parametrize("side", [98, 518])
def test_the_gpu_depth_matches_transformers_on_its_own_state_dict(ctx, side):
    """transformers' DepthAnythingForDepthEstimation (random parameters, see
    tests/test_transformers_dav2.py) saved as safetensors, loaded, run on the
    GPU in f32: the depth within the reference's feature tolerance (max 2e-3,
    mean 5e-5, load/depth_anything_v2/reference.rs:198-244) scaled by the
    depth's largest value; at 518 pixels the embedding is used as stored."""
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers")
    from safetensors.torch import save

    from tests.test_transformers_dav2 import hf_model

    model = hf_model()
    archive = load.Archive.parse(save({k: v.contiguous() for k, v in model.state_dict().items()}))
    cfg = ir.DepthConfig.small()
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    values = load.depth_weights(archive, cfg, m, side)
    image = np.random.default_rng(side).standard_normal((side, side, 3)).astype(np.float32)
    values[m.encoder.embed.image] = image.ravel()
    got = ir.run_on_gpu(ctx, g, values)[m.depth]
    with torch.no_grad():
        want = model(pixel_values=torch.from_numpy(image).permute(2, 0, 1)[None]).predicted_depth[0].numpy().ravel()
    scale = float(np.abs(want).max())
    err = np.abs(got - want)
    assert scale > 0 and (want > 0).mean() > 0.1
    assert err.max() <= 2e-3 * scale and err.mean() <= 5e-5 * scale, (err.max(), err.mean(), scale)


def test_the_f16_model_stays_near_transformers(ctx):
    """The same comparison with f16 storage (f32 accumulation) at 518 pixels:
    every weight, the image and every activation rounded to f16 (11-bit
    significands) through 12 blocks and the decoder. The bound, 1e-2 of the
    depth's largest value at most and 1e-3 of it on average, is a few times
    the error measured on this model (max 3.0e-3, mean 1.4e-4 of the scale)."""
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers")
    from safetensors.torch import save

    from beatlm_amd import hip
    from tests.test_transformers_dav2 import hf_model

    model = hf_model()
    archive = load.Archive.parse(save({k: v.contiguous() for k, v in model.state_dict().items()}))
    cfg = ir.DepthConfig.small()
    side = 518
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    values = load.depth_weights(archive, cfg, m, side)
    image = np.random.default_rng(7).standard_normal((side, side, 3)).astype(np.float32)
    values[m.encoder.embed.image] = image.ravel()
    got = ir.run_on_gpu(ctx, g, {t: v.astype(np.float16) for t, v in values.items()}, dtype=hip.F16)[m.depth]
    with torch.no_grad():
        want = model(pixel_values=torch.from_numpy(image).permute(2, 0, 1)[None]).predicted_depth[0].numpy().ravel()
    scale = float(np.abs(want).max())
    err = np.abs(got - want)
    print(f"f16 depth at 518: max err {err.max() / scale:.2e}, mean {err.mean() / scale:.2e} of scale {scale:.3e}")
    assert scale > 0 and (want > 0).mean() > 0.1
    assert err.max() <= 1e-2 * scale and err.mean() <= 1e-3 * scale, (err.max(), err.mean(), scale)
