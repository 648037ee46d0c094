"""Seeded synthetic decode inputs: the reference's recipe and the benchmark
configurations.

``make_decode_case`` follows reference ``benchmarks/data.py:8-43``: a CPU
``torch.Generator`` seeded with ``seed``; fp32 ``randn`` for q, then k, then
v; a ``randperm`` of the physical blocks so logical and physical page order
differ; table entries at or beyond ``ceil(len/block_size)`` set to -1; cast
to dtype/device last.  ``exact_pool=True`` sizes the pool to exactly the
needed blocks (the benchmark configs), handing each sequence its slice of
the permutation.  ``k_scale`` multiplies K before the cast (long-context
config).  ``device_gen=True`` draws the tensors on the GPU instead (same
shapes, metadata and lengths, different random values), for the multi-GB
configs where CPU generation would dominate.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


def make_decode_case(*, lengths, q_heads=8, kv_heads=2, head_dim=64, block_size=16,
                     dtype=torch.float32, device="cpu", seed=42, exact_pool=False,
                     k_scale=1.0, device_gen=False):
    """Returns ``(q, k_cache, v_cache, block_table, context_lens)``."""
    assert lengths and all(x >= 0 for x in lengths)
    assert q_heads % kv_heads == 0
    bsz = len(lengths)
    max_pages = max(1, math.ceil(max(lengths) / block_size))
    used = [math.ceil(x / block_size) for x in lengths]
    num_blocks = max(1, sum(used)) if exact_pool else bsz * max_pages
    gen_dev = device if device_gen else "cpu"
    gen = torch.Generator(device=gen_dev).manual_seed(seed)
    q = torch.randn(bsz, q_heads, head_dim, generator=gen, dtype=torch.float32, device=gen_dev)
    k = _randn_cast((num_blocks, block_size, kv_heads, head_dim), gen, gen_dev, dtype, k_scale)
    v = _randn_cast((num_blocks, block_size, kv_heads, head_dim), gen, gen_dev, dtype, 1.0)
    cpu_gen = gen if not device_gen else torch.Generator(device="cpu").manual_seed(seed)
    order = torch.randperm(num_blocks, generator=cpu_gen, dtype=torch.int64)
    if exact_pool:
        table = torch.full((bsz, max_pages), -1, dtype=torch.int32)
        offset = 0
        for b, n in enumerate(used):
            table[b, :n] = order[offset:offset + n].to(torch.int32)
            offset += n
    else:
        table = order.view(bsz, max_pages).to(torch.int32)
        for b, n in enumerate(used):
            table[b, n:] = -1
    return (
        q.to(device=device, dtype=dtype).contiguous(),
        k.to(device=device).contiguous(),
        v.to(device=device).contiguous(),
        table.to(device=device).contiguous(),
        torch.tensor(lengths, dtype=torch.int32, device=device),
    )


def _randn_cast(shape, gen, gen_dev, dtype, scale):
    """fp32 randn (times scale) cast to dtype, in slices to bound fp32 memory."""
    out = torch.empty(shape, dtype=dtype, device=gen_dev)
    flat = out.view(shape[0], -1)
    step = max(1, (1 << 26) // max(1, flat.shape[1]))
    for s in range(0, shape[0], step):
        e = min(shape[0], s + step)
        chunk = torch.randn((e - s, flat.shape[1]), generator=gen, dtype=torch.float32, device=gen_dev)
        if scale != 1.0:
            chunk.mul_(scale)
        flat[s:e].copy_(chunk)
    return out


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    seed: int
    len_range: tuple[int, int] | None = None
    fixed_lengths: tuple[int, ...] | None = None
    k_scale: float = 1.0
    force_ones: int = 0
    description: str = field(default="", compare=False)

    def lengths(self) -> list[int]:
        if self.fixed_lengths is not None:
            return list(self.fixed_lengths)
        lo, hi = self.len_range
        gen = torch.Generator(device="cpu").manual_seed(10_000 + self.seed)
        lens = torch.randint(lo, hi + 1, (self.batch,), generator=gen).tolist()
        for i in range(self.force_ones):
            lens[(i * self.batch) // max(1, self.force_ones)] = 1
        return lens

    def make(self, device="cpu", device_gen=False, lengths=None):
        return make_decode_case(lengths=lengths or self.lengths(), q_heads=self.q_heads,
                                kv_heads=self.kv_heads, head_dim=self.head_dim,
                                block_size=self.block_size, dtype=self.dtype, device=device,
                                seed=self.seed, exact_pool=True, k_scale=self.k_scale,
                                device_gen=device_gen)


CONFIGS: dict[str, DecodeConfig] = {
    "cfg1": DecodeConfig("cfg1", 4, 8, 2, 64, 16, torch.float16, 42,
                         fixed_lengths=(17, 100, 255, 512),
                         description="reference CPU-path config, pool = the 57 needed blocks"),
    "cfg2": DecodeConfig("cfg2", 32, 32, 8, 128, 16, torch.bfloat16, 1, len_range=(512, 4096),
                         description="Qwen3-8B-shaped decode"),
    "cfg3": DecodeConfig("cfg3", 64, 28, 4, 128, 16, torch.bfloat16, 2, len_range=(1, 8192),
                         force_ones=2, description="Qwen2.5-7B-shaped ragged decode"),
    "cfg4": DecodeConfig("cfg4", 8, 64, 8, 128, 16, torch.bfloat16, 3,
                         len_range=(32768, 131072), k_scale=3.0,
                         description="long-context split-K decode, K x3"),
    "cfg5": DecodeConfig("cfg5", 256, 40, 8, 128, 32, torch.float16, 4, len_range=(128, 1024),
                         description="high-batch short-context decode"),
}

# Measurement-only shapes (bench.py --config), not BASELINE configs: cfg2's
# lengths with 64 query heads, the group size 8 of cfg4 at cfg2's bytes per
# kv-head, for the MFMA-versus-VALU comparison.
EXTRA_CONFIGS: dict[str, DecodeConfig] = {
    "cfg2-g8": DecodeConfig("cfg2-g8", 32, 64, 8, 128, 16, torch.bfloat16, 1, len_range=(512, 4096),
                            description="cfg2 lengths with 64 q-heads (group 8)"),
}


def get_config(name: str) -> DecodeConfig:
    """A BASELINE config (CONFIGS) or a measurement-only one (EXTRA_CONFIGS)."""
    if name in CONFIGS:
        return CONFIGS[name]
    if name in EXTRA_CONFIGS:
        return EXTRA_CONFIGS[name]
    raise KeyError(f"unknown config {name!r}; known: {sorted(CONFIGS) + sorted(EXTRA_CONFIGS)}")


def algorithmic_bytes(lengths, batch, q_heads, kv_heads, head_dim, block_size, elem_bytes) -> int:
    """K+V of valid tokens + q + out + lengths + used table entries.

    Excludes split partials, re-reads and padding slots.
    """
    toks = sum(max(0, int(x)) for x in lengths)
    pages = sum(math.ceil(max(0, int(x)) / block_size) for x in lengths)
    return (toks * 2 * kv_heads * head_dim * elem_bytes + 2 * batch * q_heads * head_dim * elem_bytes
            + 4 * batch + 4 * pages)


def algorithmic_flops(lengths, q_heads, head_dim) -> int:
    return 4 * q_heads * head_dim * sum(max(0, int(x)) for x in lengths)


# ----------------------------------------------------------------------------
# Paged MLA decode inputs
# ----------------------------------------------------------------------------


def make_mla_case(*, lengths, q_len=1, heads=16, nope_dim=128, latent_dim=512, rope_dim=64, value_dim=128,
                  block_size=64, dtype=torch.bfloat16, device="cpu", seed=7, num_indices=None,
                  device_gen=False):
    """Seeded paged-MLA decode inputs, the recipe of the reference's MLA
    benchmarks (``benchmarks/bench_attention_primitives.py:47-51``): fp32
    ``randn`` q_nope, q_rope, latent and rope keys; ``w_uk`` scaled by
    ``1/sqrt(Dn)`` and ``w_uv`` by ``1/sqrt(Dc)``; cast to dtype last.

    The cache ``[N, P, Dc+Dr]`` holds exactly the needed pages in a random
    physical order, table entries past each sequence's pages are -1, and
    query t of sequence b sits at absolute position ``len - q_len + t``.
    With ``num_indices`` an index list ``[B, T, K]`` of distinct visible
    tokens per query (padded with -1) is returned as well.

    Returns a dict with q_nope, q_rope, cache, table, lens, positions, w_uk,
    w_uv, indices (or None).
    """
    bsz = len(lengths)
    P = block_size
    max_pages = max(1, math.ceil(max(lengths) / P))
    used = [math.ceil(x / P) for x in lengths]
    nblocks = max(1, sum(used))
    W = latent_dim + rope_dim
    gen_dev = device if device_gen else "cpu"
    gen = torch.Generator(device=gen_dev).manual_seed(seed)
    f32 = dict(generator=gen, dtype=torch.float32, device=gen_dev)
    q_nope = torch.randn(bsz, q_len, heads, nope_dim, **f32)
    q_rope = torch.randn(bsz, q_len, heads, rope_dim, **f32)
    cache = _randn_cast((nblocks, P, W), gen, gen_dev, dtype, 1.0)
    w_uk = torch.randn(heads, nope_dim, latent_dim, **f32) / math.sqrt(nope_dim)
    w_uv = torch.randn(heads, value_dim, latent_dim, **f32) / math.sqrt(latent_dim)
    cpu_gen = torch.Generator(device="cpu").manual_seed(seed + 1)
    order = torch.randperm(nblocks, generator=cpu_gen, dtype=torch.int64)
    table = torch.full((bsz, max_pages), -1, dtype=torch.int32)
    offset = 0
    for b, n in enumerate(used):
        table[b, :n] = order[offset:offset + n].to(torch.int32)
        offset += n
    lens = torch.tensor(lengths, dtype=torch.int32)
    positions = torch.tensor([[max(0, x - q_len + t) for t in range(q_len)] for x in lengths],
                             dtype=torch.int32).view(bsz, q_len)
    indices = None
    if num_indices is not None:
        indices = torch.full((bsz, q_len, num_indices), -1, dtype=torch.int32)
        for b in range(bsz):
            for t in range(q_len):
                visible = min(lengths[b], int(positions[b, t]) + 1)
                if visible > 0:
                    pick = torch.randperm(visible, generator=cpu_gen)[:num_indices]
                    indices[b, t, :pick.numel()] = pick.to(torch.int32)
    out = dict(q_nope=q_nope, q_rope=q_rope, cache=cache, table=table, lens=lens, positions=positions,
               w_uk=w_uk, w_uv=w_uv, indices=indices)
    for key, val in out.items():
        if val is None:
            continue
        if val.is_floating_point():
            val = val.to(dtype)
        out[key] = val.to(device).contiguous()
    return out


def mla_attend_bytes(lengths, q_len, heads, latent_dim, rope_dim, block_size, elem_bytes, num_indices=None) -> int:
    """Algorithmic HBM bytes of one latent-attention call: every visible
    cache row once per query row (or each listed row once), the absorbed
    query and rope query, the output, lengths, positions and used table
    entries.  Assumes queries at the last q_len positions (causal)."""
    W = latent_dim + rope_dim
    rows = 0
    for x in lengths:
        for t in range(q_len):
            vis = max(0, x - q_len + t + 1) if x >= q_len else x
            rows += min(vis, num_indices) if num_indices is not None else vis
    bsz = len(lengths)
    per_row_q = heads * (latent_dim + rope_dim + latent_dim) * elem_bytes
    table = sum(math.ceil(x / block_size) for x in lengths) * 4
    idx = bsz * q_len * num_indices * 4 if num_indices is not None else 0
    return rows * W * elem_bytes + bsz * q_len * per_row_q + 4 * bsz + 4 * bsz * q_len + table + idx


@dataclass(frozen=True)
class MlaConfig:
    """A paged-MLA decode workload (DeepSeek-V3 attention shapes: 128 heads,
    Dn 128, Dc 512, Dr 64, Dv 128)."""
    name: str
    description: str
    batch: int
    heads: int
    len_range: tuple
    seed: int
    block_size: int = 64
    nope_dim: int = 128
    latent_dim: int = 512
    rope_dim: int = 64
    value_dim: int = 128
    dtype: torch.dtype = torch.bfloat16

    def lengths(self):
        gen = torch.Generator().manual_seed(20_000 + self.seed)
        lo, hi = self.len_range
        return torch.randint(lo, hi + 1, (self.batch,), generator=gen).tolist()

    def make(self, device="cpu", device_gen=False):
        return make_mla_case(lengths=self.lengths(), q_len=1, heads=self.heads, nope_dim=self.nope_dim,
                             latent_dim=self.latent_dim, rope_dim=self.rope_dim, value_dim=self.value_dim,
                             block_size=self.block_size, dtype=self.dtype, device=device, seed=self.seed,
                             device_gen=device_gen)


MLA_CONFIGS = {
    "mla-h128": MlaConfig("mla-h128", "DeepSeek-V3 MLA decode, all 128 heads on one GPU, B32, len U[1024,4096], P64",
                          batch=32, heads=128, len_range=(1024, 4096), seed=11),
    "mla-h16": MlaConfig("mla-h16", "DeepSeek-V3 MLA decode, 16-head share (TP8), B128, len U[1024,4096], P64",
                         batch=128, heads=16, len_range=(1024, 4096), seed=12),
}
