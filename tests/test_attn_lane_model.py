"""CPU model of the paged-attention kernel's wavefront data flow (csrc/attn.hip), lane by lane.

The kernel's correctness rests on how it places data in the 16x16x32 MFMA operands: S^T = K Q^T
from the K pages as they lie, the probabilities kept in the lanes that computed them and fed back
as the B operand of O^T = V^T P^T, whose reduction index j = 8 (l/16) + i stands for key
4 (l/16) + i (i < 4) or 16 + 4 (l/16) + i - 4 (i >= 4) of a 32-key block, read from transposed V
pages. This test executes that data flow with numpy (the MFMA by its documented operand layouts:
lane l holds A[l % 16][8 (l/16) + i], B[8 (l/16) + i][l % 16], and D[4 (l/16) + i][l % 16]) for
prefill tiles and for the decode path's four-wavefront split and merge, on paged, GQA, ragged
batches, and compares with the attention oracle. It pins the layout reasoning on the CPU; the
GPU tests check the compiled kernel itself."""
import numpy as np
import torch

from oracle.attn_oracle import paged_attention_ref

LANES = np.arange(64)
R, QD = LANES % 16, LANES // 16


def bf16(x):
    return torch.from_numpy(np.asarray(x, np.float32)).bfloat16().float().numpy()


def mfma(A, B, C):
    """A, B: [64, 8] per-lane operands; C: [64, 4] per-lane accumulator."""
    Am = np.zeros((16, 32), np.float64)
    Bm = np.zeros((32, 16), np.float64)
    for l in range(64):
        Am[l % 16, 8 * (l // 16):8 * (l // 16) + 8] = A[l]
        Bm[8 * (l // 16):8 * (l // 16) + 8, l % 16] = B[l]
    Dm = Am @ Bm
    out = C.astype(np.float64).copy()
    for l in range(64):
        for i in range(4):
            out[l, i] += Dm[4 * (l // 16) + i, l % 16]
    return out.astype(np.float32)


def wave(q, kc, vt, bt_row, kv_len, q_len, q_start, tok0, kvh, group, blocks, scale_log2):
    """One wavefront: returns (m, l_row, O^T lanes [64, D/16, 4]) after the given key blocks."""
    D = q.shape[-1]
    page, Hkv = kc.shape[1], kc.shape[2]
    tok_r = tok0 + R // group
    valid = tok_r < q_len
    head_r = kvh * group + R % group
    qpos = kv_len - q_len + tok_r
    qop = np.zeros((64, D // 32, 8), np.float32)
    for l in range(64):
        if valid[l]:
            for s in range(D // 32):
                qop[l, s] = q[q_start + tok_r[l], head_r[l], 32 * s + 8 * QD[l]:][:8]
    m = np.full(64, -np.inf, np.float32)
    lsum = np.zeros(64, np.float32)
    o = np.zeros((64, D // 16, 4), np.float32)
    for kb in blocks:
        key0 = 32 * kb
        st = []
        for t in range(2):
            kop = np.zeros((64, D // 32, 8), np.float32)
            for l in range(64):
                kcl = min(key0 + 16 * t + R[l], kv_len - 1)
                pg = bt_row[kcl // page]
                for s in range(D // 32):
                    kop[l, s] = kc[pg, kcl % page, kvh, 32 * s + 8 * QD[l]:][:8]
            acc = np.zeros((64, 4), np.float32)
            for s in range(D // 32):
                acc = mfma(kop[:, s], qop[:, s], acc)
            st.append(acc)
        vop = np.zeros((2, 64, D // 16, 4), np.float32)
        for h in range(2):
            for l in range(64):
                g = key0 + 16 * h + 4 * QD[l]
                ga = g if g < kv_len else ((kv_len - 1) & ~3)
                pg = bt_row[ga // page]
                for c in range(D // 16):
                    vals = vt[pg, kvh, 16 * c + R[l], ga % page:ga % page + 4].copy()
                    vals[max(0, kv_len - g):] = 0.0
                    vop[h, l, c] = vals
        sc = np.full((64, 2, 4), -np.inf, np.float32)
        for t in range(2):
            for i in range(4):
                key = key0 + 16 * t + 4 * QD + i
                ok = valid & (key < kv_len) & (key <= qpos)
                sc[:, t, i] = np.where(ok, st[t][:, i] * scale_log2, -np.inf)
        mx = sc.reshape(64, 8).max(1)
        mx = np.maximum(mx, mx[LANES ^ 16])
        mx = np.maximum(mx, mx[LANES ^ 32])
        m_new = np.maximum(m, mx)
        m_use = np.where(m_new == -np.inf, 0.0, m_new).astype(np.float32)
        alpha = np.exp2(m - m_use)
        pr = np.exp2(sc - m_use[:, None, None])
        lsum = lsum * alpha + pr.reshape(64, 8).sum(1)
        m = m_new
        pop = bf16(pr.reshape(64, 8))   # [tile 0 keys 4qd+i, tile 1 keys 16+4qd+i]
        for c in range(D // 16):
            a = bf16(np.concatenate([vop[0, :, c], vop[1, :, c]], 1))
            o[:, c] = mfma(a, pop, o[:, c] * alpha[:, None])
    l_row = lsum + lsum[LANES ^ 16]
    l_row = l_row + l_row[LANES ^ 32]
    return m, l_row, o


def model_attention(q, kc, vt, qsl, kv_lens, bt, scale):
    T, H, D = q.shape
    Hkv = kc.shape[2]
    group = H // Hkv
    tpw = 16 // group
    out = np.zeros_like(q)
    sl2 = np.float32(scale * 1.4426950408889634)
    for b in range(len(kv_lens)):
        q_len, kv_len, q_start = qsl[b + 1] - qsl[b], kv_lens[b], qsl[b]
        for kvh in range(Hkv):
            if q_len == 1:   # decode: four wavefronts take every fourth block, merged
                nblk = -(-kv_len // 32)
                parts = [wave(q, kc, vt, bt[b], kv_len, 1, q_start, 0, kvh, group,
                              range(w, nblk, 4), sl2) for w in range(4)]
                for row in range(group):
                    lane = row   # any lane with l % 16 == row holds the row's stats
                    M = max(p[0][lane] for p in parts)
                    Mu = 0.0 if M == -np.inf else M
                    L = sum(np.exp2(p[0][lane] - Mu) * p[1][lane] for p in parts)
                    acc = np.zeros(D, np.float32)
                    for p in parts:
                        od = np.zeros(D, np.float32)
                        for l in range(64):
                            if l % 16 == row:
                                for c in range(D // 16):
                                    od[16 * c + 4 * (l // 16):][:4] = p[2][l, c]
                        acc += np.exp2(p[0][lane] - Mu) * od
                    out[q_start, kvh * group + row] = acc / (L if L != 0 else 1.0)
            elif q_len >= 2:
                for tok0 in range(0, q_len, tpw):
                    last = min(tok0 + tpw, q_len) - 1
                    kv_end = kv_len - q_len + last + 1
                    m, l_row, o = wave(q, kc, vt, bt[b], kv_len, q_len, q_start, tok0, kvh,
                                       group, range(-(-kv_end // 32)), sl2)
                    for l in range(64):
                        tok = tok0 + R[l] // group
                        if tok >= q_len:
                            continue
                        inv = 1.0 / (l_row[l] if l_row[l] != 0 else 1.0)
                        for c in range(D // 16):
                            d0 = 16 * c + 4 * QD[l]
                            out[q_start + tok, kvh * group + R[l] % group, d0:d0 + 4] = \
                                o[l, c] * inv
    return out


def test_lane_model_matches_oracle():
    g = torch.Generator().manual_seed(0)
    H, Hkv, D, page = 8, 2, 64, 8          # GQA group 4: four tokens per wavefront
    q_lens, kv_lens = [5, 1, 1, 19, 0], [37, 70, 3, 19, 0]
    num_pages = 40
    kc = (torch.randn(num_pages, page, Hkv, D, generator=g)).bfloat16()
    vc = (torch.randn(num_pages, page, Hkv, D, generator=g)).bfloat16()
    # unused cache slots hold NaN: masking must keep them out of every result
    perm = (torch.randperm(num_pages - 1, generator=g) + 1).tolist()
    bt = torch.zeros(len(kv_lens), 16, dtype=torch.int32)
    used = set()
    for b, n in enumerate(kv_lens):
        for j in range(-(-n // page)):
            bt[b, j] = perm.pop()
            used.add(int(bt[b, j]))
    for b, n in enumerate(kv_lens):
        if n % page:
            last = int(bt[b, (n - 1) // page])
            kc[last, n % page:] = float("nan")
            vc[last, n % page:] = float("nan")
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    q = torch.randn(qsl[-1], H, D, generator=g).bfloat16()
    scale = D ** -0.5
    ref = paged_attention_ref(q.float(), kc.float(), vc.float(), qsl, kv_lens, bt, scale)
    vt = vc.float().permute(0, 2, 3, 1).contiguous().numpy()   # [num_pages, Hkv, D, page]
    out = model_attention(q.float().numpy(), kc.float().numpy(), vt, qsl, kv_lens, bt.numpy(),
                          scale)
    assert np.isfinite(out).all()
    err = np.abs(out - ref.numpy()).max()
    assert err <= 1e-2, err
