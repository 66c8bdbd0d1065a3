"""Attention masks of the reference graphs, as compact group tables.

The reference builds dense additive [T, T] masks (0 = keep, lowest() = block)
once per configuration and streams them through every layer. The device
kernel takes the same blocked set as a group table instead: every token gets
a small group id, and allow[qg, kg] says whether a query of group qg may see a
key of group kg (VLA_MASK_GROUPS). ``dense()`` turns either form back into the
reference's additive array, which is what the parity tests feed the reference.
"""

from __future__ import annotations

import numpy as np

LOWEST = np.finfo(np.float32).min  # std::numeric_limits<float>::lowest()


def dense(keep: np.ndarray) -> np.ndarray:
    """Boolean keep matrix -> the reference's additive mask."""
    return np.where(keep, np.float32(0.0), LOWEST).astype(np.float32)


def keep_from_groups(q_group, k_group, allow) -> np.ndarray:
    G = int(round(np.sqrt(np.asarray(allow).size)))
    A = np.asarray(allow, bool).reshape(G, G)
    return A[np.asarray(q_group)[:, None], np.asarray(k_group)[None, :]]


def octo_block_causal(n_task=16, tok_primary=256, tok_wrist=64, n_readout=1, wnd=2,
                      timestep_mask=None, wrist=True, repeat_task=False):
    """Octo's block-causal mask (src/models/octo/octo_transformer.cpp:106-142).

    Token groups: 0 task (timestep -1), then per timestep t: 1 obs_primary,
    2 obs_wrist, 3 obs_language (the repeated task tokens, present when
    repeat_task), 4 readout. attends(): task -> task only; anyone -> task;
    -> obs_* when tj <= ti; readout -> readout when tj <= ti. Keys of padded
    timesteps are blocked for primary (and wrist) tokens.

    Returns (q_group, k_group, allow) with one group per (kind, timestep,
    pad) combination, and the token count.
    """
    tsm = np.ones(wnd, np.uint8) if timestep_mask is None else np.asarray(timestep_mask, np.uint8)
    kinds = [(1, tok_primary), (2, tok_wrist)] + ([(3, n_task)] if repeat_task else []) + [(4, n_readout)]
    grp, ts, pad = [0] * n_task, [-1] * n_task, [1] * n_task
    for t in range(wnd):
        for g, n in kinds:
            p = int(tsm[t]) if g == 1 else (int(wrist and tsm[t]) if g == 2 else 1)
            grp += [g] * n
            ts += [t] * n
            pad += [p] * n
    # group id per distinct (grp, ts, pad)
    combos = sorted(set(zip(grp, ts, pad)))
    gid = {c: i for i, c in enumerate(combos)}
    ids = np.array([gid[c] for c in zip(grp, ts, pad)], np.uint8)

    def attends(gi, ti, gj, tj):
        if gi == 0:
            return gj == 0
        if gj == 0:
            return True
        if gj <= 3:
            return tj <= ti
        return gi == 4 and gj == 4 and tj <= ti

    G = len(combos)
    allow = np.zeros((G, G), np.uint8)
    for a, (gi, ti, _pi) in enumerate(combos):
        for b, (gj, tj, pj) in enumerate(combos):
            allow[a, b] = 1 if (attends(gi, ti, gj, tj) and pj) else 0
    return ids, ids.copy(), allow.reshape(-1), len(ids)


def smolvla_prefix_lm(n_img=128, n_lang=48, lang_mask=None):
    """SmolVLA's prefix-LM mask (src/models/smolvla/smolvla_model.cpp:222-234).

    Prefix = images, language, one state token; att = 1 only for the state
    token; keep[i, j] = att[j] <= att[i] and pad[i] and pad[j].
    """
    lm = np.ones(n_lang, np.uint8) if lang_mask is None else np.asarray(lang_mask, np.uint8)
    n = n_img + n_lang + 1
    pad = np.concatenate([np.ones(n_img, np.uint8), lm, np.ones(1, np.uint8)])
    att = np.zeros(n, np.uint8)
    att[-1] = 1
    ids = (att * 2 + pad).astype(np.uint8)  # groups 0..3 = (att, pad)
    allow = np.zeros((4, 4), np.uint8)
    for a in range(4):
        for b in range(4):
            ai, pi = divmod(a, 2)
            aj, pj = divmod(b, 2)
            allow[a, b] = 1 if (aj <= ai and pi and pj) else 0
    return ids, ids.copy(), allow.reshape(-1), pad


def smolvla_denoise(pad_prefix, chunk=50):
    """The action expert's self-attention mask (smolvla_model.cpp:241-249):
    suffix query i sees prefix key j when pad[j], suffix key j when j <= i.

    Groups: 0 = blocked prefix key, 1 = kept prefix key, 2 + i = suffix token i.
    """
    pad = np.asarray(pad_prefix, np.uint8)
    n_prefix = len(pad)
    G = 2 + chunk
    k_group = np.concatenate([pad.astype(np.uint8), (2 + np.arange(chunk)).astype(np.uint8)])
    q_group = (2 + np.arange(chunk)).astype(np.uint8)
    allow = np.zeros((G, G), np.uint8)
    for i in range(chunk):
        allow[2 + i, 1] = 1
        allow[2 + i, 2:2 + i + 1] = 1
    return q_group, k_group, allow.reshape(-1), n_prefix + chunk
