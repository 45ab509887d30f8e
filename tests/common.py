"""Shared helpers of the test suite: the tiny configurations of the
reference's tests (crates/omg-wgpu/tests/reference.rs:40-104), engines and
oracles built on identical seeded weights, and the comparison measures the
reference's tests use."""
from __future__ import annotations

import numpy as np

import grande_amd as g
import oracle


def gemma3_tiny(**over) -> str:
    """reference.rs:40-65: vocab 40, d 64, 3 layers, 2 heads over 1 KV head,
    head_dim 256, ff 96, window 6, sliding/global/sliding, (1 + w) norms."""
    kw = dict(vocab=40, d=64, layers=3, heads=2, kv_heads=1, head_dim=256, ff=96, window=6,
              sliding=[True, False, True], norm_offset=None)
    kw.update(over)
    return g.config_json(**kw)


def gguf_tiny(heads: int = 4, kv_heads: int = 1, **over) -> str:
    """A GGUF-style tiny Gemma 3 (norm offset folded in, norms around 1),
    quantized weights; heads / kv_heads vary the GQA grouping."""
    kw = dict(vocab=64, d=64, layers=4, heads=heads, kv_heads=kv_heads, head_dim=256, ff=96, window=5,
              sliding=[True, False, True, False], norm_offset=0.0)
    kw.update(over)
    return g.config_json(**kw)


def gemma4_tiny(heads: int = 4, kv_heads: int = 1, **over) -> str:
    """reference.rs:66-104: vocab 64, d 64, 4 layers, head_dim 256 / 512
    (sliding / global), ff 96, 96, 192, 192, layers 2 and 3 reading the K/V
    of layers 0 and 1, RoPE on 256 / 128 dims, window 5, V norm, per-layer
    inputs of 32, softcap 30; (heads, kv_heads) = (8, 2) is the GQA variant."""
    kw = dict(vocab=64, d=64, layers=4, heads=heads, kv_heads=kv_heads, head_dim=256, global_head_dim=512, ff=96,
              double_wide_mlp=True, shared_kv_layers=2, window=5, sliding=[True, False, True, False],
              partial_rotary_global=0.25, per_layer_dim=32, softcap=30.0)
    kw.update(over)
    return g.gemma4_config_json(**kw)


def build(cfg: str, seed: int, linear: int, embed: int, capacity: int = 64, max_rows: int = 16,
          oracle_models: bool = True):
    """(engine, plain f32 oracle, GPU-rounding oracle, weights) on identical
    seeded weights (reference.rs:106-139)."""
    w = g.Weights.synth(cfg, seed, linear, embed)
    eng = g.Engine.new(w, capacity, max_rows)
    if not oracle_models:
        return eng, None, None, w
    ts = list(w.tensors())
    return eng, oracle.Model(cfg, ts), oracle.Model(cfg, ts, gpu_rounding=True), w


def max_abs_diff(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def rel_diff(got, exp) -> float:
    """reference.rs:399-403: max |got - exp| / max(max |exp|, 1)."""
    exp = np.asarray(exp, np.float64)
    return max_abs_diff(got, exp) / max(float(np.max(np.abs(exp))), 1.0)


def assert_close(a, b, what: str, tol: float = 1e-4) -> None:
    """reference.rs:720-735: max |a - b| <= tol * max(max |a|, 1)."""
    a = [np.asarray(x) for x in a]
    b = [np.asarray(x) for x in b]
    assert len(a) == len(b), f"{what}: row count"
    worst = max(max_abs_diff(x, y) for x, y in zip(a, b))
    scale = max(float(np.max(np.abs(x))) for x in a)
    assert worst <= tol * max(scale, 1.0), f"{what}: max |d| {worst:e} at scale {scale:e}"


def oracle_rows(model: oracle.Model, prefix, branches) -> list[list[np.ndarray]]:
    """The oracle's final hidden rows at each branch's wanted positions."""
    ids, pos, seq = oracle.pack_single(prefix, branches)
    hidden = model.forward(ids, pos, seq)
    out, idx = [], len(prefix)
    for b in branches:
        out.append([hidden[idx + w] for w in b.want])
        idx += len(b.tokens)
    return out


def random_request(rng: np.random.Generator, vocab: int, state: int, nbranches: int, branch_tokens: int,
                   want_last: bool = True):
    prefix = rng.integers(0, vocab, state).tolist()
    branches = [g.BranchTokens(rng.integers(0, vocab, branch_tokens).tolist(),
                               [branch_tokens - 1] if want_last else list(range(branch_tokens)))
                for _ in range(nbranches)]
    return prefix, branches


def tiled_oracle(cfg: str, tensors, capacity: int) -> oracle.Model:
    """The f16-rounding oracle with the HIP attention kernel's own rounding
    points too (32-key tiles, lazily moved whole-power-of-two max, P in f16,
    f16 chunk partials at the engine's chunk lengths for this capacity:
    256 keys on sliding layers, max(384 keys, an eighth of the cache) on
    global ones)."""
    kt = 32
    cap_pad = (capacity + 63) // 64 * 64
    return oracle.Model(cfg, tensors, gpu_rounding=True).set_attention_tiles(
        kt, 256 // kt, max(384 // kt, (cap_pad // kt + 7) // 8))


def worst_rel(a, b) -> float:
    """Largest rel_diff over matching rows of two [branch][row] lists."""
    return max(rel_diff(x, y) for oa, ob in zip(a, b) for x, y in zip(oa, ob))


def rounding_spread(cfg: str, tensors, prefix, branches, capacity: int):
    """Rows of the three CPU forwards that differ only in where they round
    (plain f32; f16 operands as the reference GPU path; f16 operands plus
    the flash kernel's attention rounding) and the largest distance between
    any two of them: how far legitimate f16 implementations of this
    configuration can sit apart."""
    f32 = oracle_rows(oracle.Model(cfg, tensors), prefix, branches)
    f16 = oracle_rows(oracle.Model(cfg, tensors, gpu_rounding=True), prefix, branches)
    tiled = oracle_rows(tiled_oracle(cfg, tensors, capacity), prefix, branches)
    spread = max(worst_rel(f32, f16), worst_rel(f32, tiled), worst_rel(f16, tiled))
    return f32, f16, tiled, spread
