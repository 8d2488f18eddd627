"""Helpers shared by the GPU parity tests: device copies, the arena loader and the attention
check against the oracle (max-abs 1e-4, rel-L2 1e-5; K/V pages bit-exact)."""

import sys

import numpy as np
import torch

from cases import rel_l2
from nanollvm_amd import Attention, KvCacheArena, RMSNorm, RotaryEmbedding
from oracle import oracle as O

MAX_ABS = 1e-4
REL_L2 = 1e-5
EPS = 1e-6


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def load_arena(ctx, case):
    wl = case.wl
    if case.paged:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
    else:
        arena = KvCacheArena(ctx, 1, 2, 16, wl.hkv, wl.d)
    return arena


def check_attention(ctx, case, name, fused_rope=None):
    wl = case.wl
    say(f"{name}: tokens={wl.tokens} hq={wl.hq} hkv={wl.hkv} d={wl.d} W={wl.window}")
    arena = load_arena(ctx, case)
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
        if fused_rope is None:
            out = attn.forward(dev(case.q), dev(case.k), dev(case.v), ctx)
            want, kc, vc = case.oracle(threads=8)
        else:
            rope, table = fused_rope
            q_out = torch.empty(case.q.shape, dtype=torch.float32, device="cuda")
            k_out = torch.empty(case.k.shape, dtype=torch.float32, device="cuda")
            out = attn.forward_with_rope(rope, wl.meta.positions, dev(case.q), dev(case.k),
                                         dev(case.v), ctx, q_out=q_out, k_out=k_out)
            qr, kr = O.rope_forward(table, wl.meta.positions, case.q, case.k)
            torch.cuda.synchronize()
            assert np.array_equal(bits(q_out.cpu().numpy()), bits(qr)), "rotated q not bit-exact"
            assert np.array_equal(bits(k_out.cpu().numpy()), bits(kr)), "rotated k not bit-exact"
            case.q, case.k = qr, kr
            want, kc, vc = case.oracle(threads=8)
        ctx.sync()
        got = out.cpu().numpy()
        err = float(np.max(np.abs(got - want))) if got.size else 0.0
        rl2 = rel_l2(got, want)
        say(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e}")
        assert np.all(np.isfinite(got)), "non-finite output"
        assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)
        if case.paged:
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(kc)), "K pages differ"
            assert np.array_equal(bits(arena.get_value_cache(0)), bits(vc)), "V pages differ"
    finally:
        ctx.clear()
        arena.close()


def torch_view(ptr, count):
    """A float32 torch tensor over device memory the library owns (no copy)."""

    class _Cai:
        pass

    obj = _Cai()
    obj.__cuda_array_interface__ = {"shape": (count,), "typestr": "<f4", "data": (ptr, False),
                                    "version": 2, "strides": None}
    return torch.as_tensor(obj, device="cuda")


def arena_views(arena, layer=0):
    """Device views of one layer's K and V pages, [num_blocks, block_size * Hkv * d] each."""
    k_ptr, v_ptr, nbytes = arena.device_ptrs(layer)
    n = nbytes // 4
    nb = arena.num_blocks
    return torch_view(k_ptr, n).view(nb, -1), torch_view(v_ptr, n).view(nb, -1)


def fill_normal(arena, seed, layer=0):
    """Seeded N(0, 1) pages, written on the device."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for t in arena_views(arena, layer):
        flat = t.view(-1)
        for s in range(0, flat.numel(), 1 << 28):
            flat[s:s + (1 << 28)].normal_(generator=g)
    torch.cuda.synchronize()


def _norm_heads(x, w, one_plus):
    return O.rms_norm(x.reshape(-1, x.shape[-1]), w, EPS, one_plus).reshape(x.shape)


def check_fused(ctx, case, name, q_w, k_w, one_plus=False, v_norm=False, max_pos=None,
                theta=1e4, outputs=True, norms=True, twin=False):
    """The per-head norms + RoPE + Attention.forward chain through nva_norm_rope_attention_forward
    against the oracle chain (normHeads, RoPE, Attention.forward): rotated q/k (when `outputs`)
    and every page byte bit-exact, attention within the bar.  norms=False passes no q/k norm at
    all (RoPE only); outputs=False passes no q_out/k_out.  twin (with outputs=False): the same
    call again with q_out/k_out given must return bit-identical attention and the oracle's
    rotated q, bit for bit (whether the caller asks for the rotated rows changes nothing)."""
    wl = case.wl
    say(f"{name}: tokens={wl.tokens} hq={wl.hq} hkv={wl.hkv} d={wl.d} W={wl.window} "
        f"bs={wl.block_size} one_plus={one_plus} v_norm={v_norm} outputs={outputs}")
    max_pos = max_pos or 512
    table = O.rope_table(wl.d, max_pos, theta)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, max_pos, theta, cos_sin=table)
    if case.paged:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
    else:
        arena = KvCacheArena(ctx, 1, 2, 16, wl.hkv, wl.d)
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
        qn = RMSNorm(None if q_w is None else dev(q_w), EPS, one_plus) if norms else None
        kn = RMSNorm(None if k_w is None else dev(k_w), EPS, one_plus) if norms else None
        vn = RMSNorm.weightless(EPS) if v_norm else None
        q_out = torch.empty(case.q.shape, dtype=torch.float32, device="cuda") if outputs else None
        k_out = torch.empty(case.k.shape, dtype=torch.float32, device="cuda") if outputs else None
        q_in, k_in, v_in = case.q, case.k, case.v
        out = attn.forward_with_norm_rope(rope, wl.meta.positions, dev(case.q), dev(case.k),
                                          dev(case.v), ctx, q_norm=qn, k_norm=kn, v_norm=vn,
                                          q_out=q_out, k_out=k_out)
        # Oracle chain: normHeads(q), normHeads(k) [, vNorm(v)], RoPE, Attention.forward.
        nq = _norm_heads(case.q, q_w, one_plus) if norms else case.q
        nk = _norm_heads(case.k, k_w, one_plus) if norms else case.k
        qr, kr = O.rope_forward(table, wl.meta.positions, nq, nk)
        torch.cuda.synchronize()
        if outputs:
            assert np.array_equal(bits(q_out.cpu().numpy()), bits(qr)), "q not bit-exact"
            assert np.array_equal(bits(k_out.cpu().numpy()), bits(kr)), "k not bit-exact"
        case.q, case.k = qr, kr
        if v_norm:
            case.v = _norm_heads(case.v, None, False)
        want, kc, vc = case.oracle(threads=8)
        got = out.cpu().numpy()
        err = float(np.max(np.abs(got - want))) if got.size else 0.0
        rl2 = rel_l2(got, want)
        say(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e}")
        assert np.all(np.isfinite(got))
        assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)
        if case.paged:
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(kc)), "K pages differ"
            assert np.array_equal(bits(arena.get_value_cache(0)), bits(vc)), "V pages differ"
        if twin and not outputs:
            # Stores the same rows to the same slots again, so the pages do not change.
            q_out = torch.empty(case.q.shape, dtype=torch.float32, device="cuda")
            k_out = torch.empty(case.k.shape, dtype=torch.float32, device="cuda")
            out2 = attn.forward_with_norm_rope(rope, wl.meta.positions, dev(q_in), dev(k_in),
                                               dev(v_in), ctx, q_norm=qn, k_norm=kn,
                                               v_norm=vn, q_out=q_out, k_out=k_out)
            torch.cuda.synchronize()
            assert np.array_equal(bits(q_out.cpu().numpy()), bits(qr)), "q not bit-exact"
            assert np.array_equal(bits(out2.cpu().numpy()), bits(got)), \
                "attention differs when the rotated q/k are asked for"
    finally:
        ctx.clear()
        arena.close()
        rope.close()
