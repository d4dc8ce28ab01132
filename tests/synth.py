"""Synthetic weights and activations for the quantized-linear path, packed into the on-disk
layouts the reference loader hands to sgl_qweight_dequant* (reference src/safetensors.c:271-471).

These are data producers only (numpy, host side): they quantize an f32 weight matrix and pack
the codes the way AutoGPTQ / AutoAWQ / vLLM-Marlin / compressed-tensors / gpt-oss store them.
Parity never depends on them: whatever they pack, the dequant is checked against the oracle.

Layout facts used here (reference include/sgl/qweight.h:1-36 and src/qweight.c):
  GPTQ   qweight i32 [K/pack, N], k in slot k%pack; qzeros i32 [G', N/pack], n in slot n%pack
  AWQ    qweight i32 [K, N/8] (gemm) or [N/8, K] (gemv); column n in slot AWQ_SLOT[n&7]
  Marlin 16(k) x 64(n) tiles, word p nibble j -> (k_off, n_off) of reference src/qweight.c:241-245;
         scales/zeros permuted per reference src/qweight.c:173-191
  CT     i32 [N, K/pack], little-endian bytes, low nibble = even k; value = code - offset
  MXFP4  u8 [N, K/2] (low nibble = even k) + e8m0 u8 [N, K/32]
"""
import numpy as np

AWQ_SLOT = np.array([0, 4, 1, 5, 2, 6, 3, 7])
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def normal(seed, shape, std=1.0):
    return (rng(seed).standard_normal(shape) * std).astype(np.float32)


def to_bf16_bits(x):
    """f32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------------------
# group-wise asymmetric int quantization (GPTQ/AWQ style)
# ---------------------------------------------------------------------------------------
def quantize_groups(W, G, bits=4, g_idx=None, sym=False):
    """W f32 [N,K] -> codes u8 [N,K], zeros u8 [ng,N], scales f32 [ng,N] (fp16-exact).

    Per group: s = (max - min) / (2^bits - 1) rounded to fp16, z = clamp(round(-min/s)),
    q = clamp(round(w/s) + z).  With sym=True z = 2^(bits-1) and s = absmax / (2^(bits-1)-1)."""
    N, K = W.shape
    Ge = G if G > 0 else K
    if g_idx is None and K % Ge == 0:  # contiguous groups: the same arithmetic, vectorised
        w = W.reshape(N, K // Ge, Ge).astype(np.float32)
        qmax = (1 << bits) - 1
        if sym:
            s = (np.abs(w).max(axis=2) / ((1 << (bits - 1)) - 1)).astype(np.float16)
            s = s.astype(np.float32)
            s[s == 0] = 1.0
            z = np.full(s.shape, 1 << (bits - 1), np.float32)
        else:
            lo = np.minimum(w.min(axis=2), 0)
            hi = np.maximum(w.max(axis=2), 0)
            s = ((hi - lo) / qmax).astype(np.float16).astype(np.float32)
            s[s == 0] = 1.0
            z = np.clip(np.round(-lo / s), 0, qmax)
        q = np.clip(np.round(w / s[:, :, None]) + z[:, :, None], 0, qmax)
        return (q.reshape(N, K).astype(np.uint8), np.ascontiguousarray(z.T).astype(np.uint8),
                np.ascontiguousarray(s.T))
    if g_idx is None:
        g_idx = np.arange(K) // Ge
    ng = int(g_idx.max()) + 1
    qmax = (1 << bits) - 1
    codes = np.zeros((N, K), np.uint8)
    zeros = np.zeros((ng, N), np.uint8)
    scales = np.zeros((ng, N), np.float32)
    for g in range(ng):
        cols = np.nonzero(g_idx == g)[0]
        w = W[:, cols].astype(np.float32)
        if sym:
            amax = np.abs(w).max(axis=1)
            s = (amax / ((1 << (bits - 1)) - 1)).astype(np.float16).astype(np.float32)
            s[s == 0] = 1.0
            z = np.full(N, 1 << (bits - 1), np.float32)
        else:
            lo = np.minimum(w.min(axis=1), 0)
            hi = np.maximum(w.max(axis=1), 0)
            s = ((hi - lo) / qmax).astype(np.float16).astype(np.float32)
            s[s == 0] = 1.0
            z = np.clip(np.round(-lo / s), 0, qmax)
        q = np.clip(np.round(w / s[:, None]) + z[:, None], 0, qmax)
        codes[:, cols] = q.astype(np.uint8)
        zeros[g] = z.astype(np.uint8)
        scales[g] = s
    return codes, zeros, scales


def act_order_gidx(seed, K, G):
    """g_idx for act-order: group i // G of a seeded random permutation of K."""
    perm = rng(seed).permutation(K)
    g = np.empty(K, np.int32)
    g[perm] = np.arange(K) // G
    return g


def _pack_along(vals, bits, axis):
    """Pack u8 codes along axis (length multiple of 32/bits) into int32, value i in slot i%pack."""
    pack = 32 // bits
    v = np.moveaxis(np.asarray(vals, dtype=np.uint32), axis, -1)
    sh = v.shape[:-1] + (v.shape[-1] // pack, pack)
    v = v.reshape(sh)
    w = np.zeros(sh[:-1], np.uint32)
    for j in range(pack):
        w |= v[..., j] << np.uint32(bits * j)
    return np.moveaxis(w.view(np.int32), -1, axis)


def gptq_pack(codes, zeros, bits=4, v2=False):
    """codes [N,K] -> qweight i32 [K/pack, N]; zeros [ng,N] -> qzeros i32 [ng, N/pack]."""
    qweight = _pack_along(codes.T, bits, 0)
    z = zeros.astype(np.int32) - (1 if v2 else 0)
    z = np.where(z < 0, (1 << bits) - 1, z)  # v2 stores z-1; a zero of 0 wraps
    qzeros = _pack_along(z, bits, 1)
    return qweight, qzeros


def awq_pack(codes, zeros, transposed=False):
    """4-bit AWQ: column n in nibble AWQ_SLOT[n&7] of word n>>3."""
    N, K = codes.shape
    perm = np.empty(8, np.int64)
    perm[AWQ_SLOT] = np.arange(8)  # slot s holds column perm[s]

    def pk(v):  # v [R, N] -> [R, N/8]
        v = np.asarray(v, np.uint32).reshape(v.shape[0], N // 8, 8)[:, :, perm]
        w = np.zeros(v.shape[:2], np.uint32)
        for s in range(8):
            w |= v[:, :, s] << np.uint32(4 * s)
        return w.view(np.int32)

    qw = pk(codes.T)  # [K, N/8]
    if transposed:
        qw = np.ascontiguousarray(qw.T)  # [N/8, K]
    return qw, pk(zeros)


# ---------------------------------------------------------------------------------------
# Marlin 16x64 tiles (inverse of reference src/qweight.c:233-273)
# ---------------------------------------------------------------------------------------
def _marlin_tile_maps(bits):
    pack = 32 // bits
    tw = 64 * 16 // pack
    p = np.arange(tw)[:, None]
    j = np.arange(pack)[None, :]
    if bits == 4:
        ko = 2 * ((p >> 2) & 3) + np.where(j & 1, 8, 0) + np.where(j >= 4, 1, 0)
        no = 16 * (p & 3) + (p >> 4) + np.where(j & 2, 8, 0)
    else:
        k8 = np.array([0, 8, 1, 9])[j]
        ko = 2 * ((p >> 3) & 3) + k8
        no = 16 * ((p >> 1) & 3) + (p >> 5) + np.where(p & 1, 8, 0)
    return ko, no


def marlin_col_map(N, bits):
    """Natural column n -> (scale index, zero word column, zero slot)."""
    pack = 32 // bits
    n = np.arange(N)
    f = (n // 64) * 64 + 8 * (n & 7) + ((n % 64) >> 3)
    if pack == 8:
        jj = f & 7
        pos, gsz = (jj >> 1) + 4 * (jj & 1), 8
    else:
        jj = f & 3
        pos, gsz = ((jj & 1) << 1) | (jj >> 1), 4
    f2 = gsz * (f // gsz) + pos
    return f, f2 // pack, f2 % pack


def marlin_pack(codes, zeros, scales, bits=4, with_zeros=True):
    """Natural codes [N,K] (unsigned), zeros [ng,N], scales [ng,N] -> Marlin buffers."""
    N, K = codes.shape
    pack = 32 // bits
    ko, no = _marlin_tile_maps(bits)
    tw = ko.shape[0]
    qw = np.zeros((K // 16, (N // 64) * tw), np.uint32)
    for kt in range(K // 16):
        for nt in range(N // 64):
            c = codes[nt * 64 + no, kt * 16 + ko].astype(np.uint32)  # [tw, pack]
            w = np.zeros(tw, np.uint32)
            for jj in range(pack):
                w |= c[:, jj] << np.uint32(bits * jj)
            qw[kt, nt * tw:(nt + 1) * tw] = w
    sidx, zcol, znib = marlin_col_map(N, bits)
    sc = np.zeros_like(scales)
    sc[:, sidx] = scales
    qz = None
    if with_zeros:
        ng = zeros.shape[0]
        qz = np.zeros((ng, N // pack), np.uint32)
        for n in range(N):
            qz[:, zcol[n]] |= zeros[:, n].astype(np.uint32) << np.uint32(bits * znib[n])
        qz = qz.view(np.int32)
    return qw.view(np.int32), qz, sc


# ---------------------------------------------------------------------------------------
# compressed-tensors, MXFP4, W8
# ---------------------------------------------------------------------------------------
def ct_pack(signed_codes, bits=4):
    """signed codes [N,K] in [-2^(bits-1), 2^(bits-1)) -> i32 [N, K/pack] (code + offset)."""
    u = (signed_codes.astype(np.int32) + (1 << (bits - 1))).astype(np.uint32)
    return _pack_along(u, bits, 1)


def mxfp4_quantize(W):
    """W f32 [N,K] (K % 32 == 0) -> blocks u8 [N,K/2], e8m0 scales u8 [N,K/32].
    Per 32-block: e = floor(log2(amax/6)), element = nearest e2m1 of w / 2^e."""
    N, K = W.shape
    wb = W.reshape(N, K // 32, 32).astype(np.float64)
    amax = np.abs(wb).max(axis=2)
    e = np.floor(np.log2(np.maximum(amax, 1e-30) / 6.0)).astype(np.int64)
    e = np.clip(e, -127, 127)
    x = wb / np.exp2(e)[:, :, None]
    mag = E2M1[:8].astype(np.float64)
    idx = np.abs(np.abs(x)[..., None] - mag).argmin(axis=-1)
    code = (idx | np.where(x < 0, 8, 0)).astype(np.uint8).reshape(N, K)
    blocks = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    scales = (e + 127).astype(np.uint8)
    return blocks, scales


def quant_rows_i8(W):
    """numpy restatement of the per-row symmetric int8 quantizer semantics (f32 arithmetic)."""
    W = np.asarray(W, np.float32)
    amax = np.abs(W).max(axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = (np.float32(1.0) / scale).astype(np.float32)
    half = np.where(W >= 0, np.float32(0.5), np.float32(-0.5)).astype(np.float32)
    v = np.trunc((W * inv[:, None]).astype(np.float32) + half).astype(np.float32)
    q = np.clip(v, -127, 127).astype(np.int8)
    q[amax <= 0] = 0
    scale[amax <= 0] = 0
    return q, scale


# ---------------------------------------------------------------------------------------
# routed MoE inputs: top-k experts uniform without replacement per token,
# weights = softmax of N(0,1) logits over the k picks
# ---------------------------------------------------------------------------------------
def moe_routing(seed, T, n_exp, k):
    g = rng(seed)
    ids = np.stack([g.permutation(n_exp)[:k] for _ in range(T)]).astype(np.int32)
    logits = g.standard_normal((T, k))
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def gptq_expert(seed, N, K, G=128):
    """One GPTQ int4 g128 weight [N, K] ~ N(0, 0.02): (qweight, qzeros, scales)."""
    c, z, s = quantize_groups(normal(seed, (N, K), 0.02), G)
    qw, qz = gptq_pack(c, z)
    return qw, qz, s
