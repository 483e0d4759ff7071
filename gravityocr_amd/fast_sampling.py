"""Drop-in decode entry points with the signatures of the reference's src/fast_sampling.py, running the cached
self-speculative decode on the MI355X kernels.

``generate_speculative_natcache`` (src/fast_sampling.py:425-628) is the path: prefill the prompt into a paged KV
cache, then rounds of draft -> verify -> accept -> commit until EOS or ``max_new_tokens``. Its rounds map onto the
engine's full-draft round (gravityocr_amd/engine.py) one for one:

  * round 0 (pending = None): draft window [MASK x B] (all rows bidirectional), block[0] seeded by the prefill's
    last logit; verify [a0, d_1..d_B] causally -> ``SelfSpecDecoder.round0``.
  * rounds >= 1: draft window [pending | MASK x B] (pending row causal, block rows bidirectional); the verify of
    [pending, a0, d_1..d_B] is split in two: the pending row's K/V and argmax come from the draft's row 0 (the same
    causal row over the same cache: the engine computes it bit-identically in either forward), and the verify
    forward runs over [a0, d_1..d_B] -> ``SelfSpecDecoder.round``.
  * accept: k = first mismatch of draft vs ar_pred (ar_pred[0] = a0 always matches); committed ``new`` =
    draft[:k] + [ar_pred[k]], or draft + [bonus] on a full match; the K/V of pending + new[:-1] stays in the cache
    and new[-1] becomes the next pending token (src/fast_sampling.py:562-606). In engine terms acc = k - 1.

The model is read through the reference's protocol (src/fast_sampling.py:16-18): ``text_model`` (embed_tokens,
layers, norm), ``glm.lm_head``, ``mm_model`` (get_image_features, get_rope_index), ``processor``, ``tokenizer``,
``mask_id``, ``image_token_id``, ``bd_size``. Image preprocessing and the prompt embedding (the vision tower) run
through the model's own modules, as in the reference; everything from the prefill on runs on the kernels.

``generate_speculative_prefixcache`` (src/fast_sampling.py:262-422) runs on the same rounds: its committed ids are
those of its causal verify, i.e. AR greedy decoding, which these rounds reproduce (see its docstring).

Supported arguments: greedy decoding (``temperature == 0``), ``draft_steps == 1``, ``accept_conf == 0`` and
``full_draft=True`` -- the reference's defaults. Other values raise NotImplementedError (no silent fallback).
"""
import re
import weakref
from typing import Dict, List, Optional, Tuple

import torch

from . import kernels as K
from .diffusion import BlockDiffusionDecoder
from .engine import PAGE, GssEngine, SelfSpecDecoder
from .model import config_from_model, weights_from_model

__all__ = ["generate_speculative_natcache", "generate_speculative_prefixcache", "generate_cached",
           "teacher_force_argmax", "enable_fused_flex", "prepare_prompt"]

_MIN_CAPACITY = 4096


class _Session:
    """One model's decoder weights on the GPU, a paged KV pool for ``max_bs`` sequences and its decoders."""

    def __init__(self, model, device: torch.device, capacity: int, max_bs: int = 1):
        self.cfg = config_from_model(model)
        self.capacity, self.max_bs = capacity, max_bs
        self.eng = GssEngine(self.cfg, weights_from_model(model), max_bs=max_bs, max_len=capacity, device=device)
        self.decoders: Dict[Tuple[int, int], SelfSpecDecoder] = {}
        self.graphed: Dict[Tuple[int, int], bool] = {}
        self.diffusion: Dict[tuple, BlockDiffusionDecoder] = {}

    def diffusion_decoder(self, bs: int, bd: int, mask_id: int, threshold: float,
                          commit_causal: bool) -> BlockDiffusionDecoder:
        key = (bs, bd, mask_id, float(threshold), bool(commit_causal))
        if key not in self.diffusion:
            self.diffusion[key] = BlockDiffusionDecoder(self.eng, bd, mask_id, bs, threshold, commit_causal)
        return self.diffusion[key]

    def decoder(self, bd: int, mask_id: int) -> SelfSpecDecoder:
        key = (bd, mask_id)
        if key not in self.decoders:
            # every round commits at least 2 tokens and writes one log row
            self.decoders[key] = SelfSpecDecoder(self.eng, bd=bd, mask_id=mask_id, bs=1,
                                                 max_rounds=self.capacity // 2 + 8, softmax_rule=True)
            self.graphed[key] = False
        return self.decoders[key]


_SESSIONS: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def _session(model, device: torch.device, need: int, bs: int = 1) -> _Session:
    s = _SESSIONS.get(model)
    if s is None or s.capacity < need or s.max_bs < bs or s.eng.device != device:
        cap = max(_MIN_CAPACITY, need, 0 if s is None else s.capacity)
        cap = (cap + 1023) // 1024 * 1024
        s = _Session(model, device, cap, max(bs, 1 if s is None else s.max_bs))
        _SESSIONS[model] = s
    return s


def _model_device(model) -> torch.device:
    dev = next(model.parameters()).device
    if dev.type != "cuda":
        raise RuntimeError("the MI355X decode needs the model on a ROCm GPU (device 'cuda:N'); got " + str(dev))
    return dev


def _resize(image, max_long_side):
    from PIL import Image
    if image.mode != "RGB":
        image = image.convert("RGB")
    w, h = image.size
    if max(w, h) > max_long_side:
        s = max_long_side / max(w, h)
        image = image.resize((int(w * s), int(h * s)), Image.LANCZOS)
    return image


@torch.no_grad()
def prepare_prompt(model, image, prompt: str, max_long_side: int, device: torch.device):
    """The reference's preprocessing (src/fast_sampling.py:465-497): resize, chat template, processor, image
    features spliced over the image-token ids, M-RoPE positions. Returns (input_ids [1, P], embeddings [P, H],
    positions int32 [P, 3], next_pos)."""
    image = _resize(image, max_long_side)
    msgs = [{"role": "user", "content": [{"type": "image"}, {"type": "text", "text": prompt}]}]
    text = model.processor.apply_chat_template(msgs, add_generation_prompt=True, tokenize=False)
    enc = model.processor(text=[text], images=[image], return_tensors="pt").to(device)
    input_ids, mm_tt = enc["input_ids"], enc["mm_token_type_ids"]
    pixel_values, image_grid_thw = enc.get("pixel_values"), enc.get("image_grid_thw")
    P = input_ids.shape[1]
    tm = model.text_model
    e = tm.embed_tokens(input_ids)
    if pixel_values is not None:
        feats = model.mm_model.get_image_features(pixel_values, image_grid_thw, return_dict=True).pooler_output
        image_embeds = torch.cat(feats, dim=0).to(device)
        mm = (input_ids == model.image_token_id).unsqueeze(-1).expand_as(e)
        e = e.masked_scatter(mm, image_embeds.to(e.dtype))
    attn = torch.ones((1, P), dtype=torch.long, device=device)
    pos3, _ = model.mm_model.get_rope_index(input_ids, mm_tt, image_grid_thw=image_grid_thw, video_grid_thw=None,
                                            attention_mask=attn)
    next_pos = int(pos3.max().item()) + 1
    positions = pos3[:, 0, :].t().to(torch.int32).contiguous()          # [P, 3]
    return input_ids, e[0], positions, next_pos


def _prefill(eng: GssEngine, emb, positions, logits_rows=None, slot: int = 0):
    """Prefill one slot; 1-D positions (all three M-RoPE rows equal to 0..P-1) take the plain RoPE path."""
    P = emb.shape[0]
    ar = torch.arange(P, dtype=torch.int32, device=positions.device)
    plain = bool(((positions == ar[:, None]).all()).item())
    return eng.prefill(slot, emb, positions=None if plain else positions, logits_rows=logits_rows)


def _argmax_rows(eng: GssEngine, logits: torch.Tensor, softmax_rule: bool = False) -> torch.Tensor:
    """Greedy ids of logits [n, V] (bf16): max value, lowest index on ties; a row with a NaN gives the NaN's index
    (torch.argmax of the logits), or 0 with ``softmax_rule`` (argmax of the fp32 softmax, all NaN)."""
    n = logits.shape[0]
    out = torch.empty(n, 1, dtype=torch.int32, device=logits.device)
    step = 1024                                     # sequences per argmax launch
    for i in range(0, n, step):
        j = min(n, i + step)
        lg = logits[i:j].contiguous().view(j - i, 1, -1)
        ws = torch.zeros(K.argmax_workspace_bytes(j - i, 1, lg.shape[-1]), dtype=torch.uint8, device=logits.device)
        K.argmax_accept(lg, out[i:j], ws, flags=K.ARGMAX_SOFTMAX if softmax_rule else 0)
    return out[:, 0]


def _check_greedy(temperature, accept_conf=0.0, draft_steps=1, full_draft=True):
    """Reject the non-greedy and non-default modes this path does not implement (no silent fallback)."""
    if temperature and temperature > 0:
        raise NotImplementedError("only greedy decoding (temperature=0) runs on the MI355X path")
    if accept_conf and accept_conf > 0:
        raise NotImplementedError("accept_conf > 0 (probability-threshold acceptance) is not implemented")
    if draft_steps != 1:
        raise NotImplementedError("only draft_steps=1 (one draft forward per round) is implemented")
    if not full_draft:
        raise NotImplementedError("only full_draft=True (a0, d_1..d_B and the bonus token) is implemented")


def _decode_text(model, gen: List[int], device) -> str:
    if not gen:
        return ""
    txt = model.tokenizer.decode(torch.tensor(gen, device=device), skip_special_tokens=True)
    return re.sub(r"<think>.*?</think>\s*", "", txt, flags=re.S)


def _spec_rounds(model, image, prompt, max_new_tokens, max_long_side, bd):
    """Prompt, prefill and the full-draft rounds of the cached self-spec decode on the engine. Returns (the packed
    row of every round that counts, the decoder, the tokenizer's EOS id, the device)."""
    device = _model_device(model)
    mask_id = int(model.mask_id)
    eos_id = model.tokenizer.eos_token_id
    input_ids, emb, positions, next_pos = prepare_prompt(model, image, prompt, max_long_side, device)
    P = input_ids.shape[1]
    # capacity: prompt + budget + the last round's overshoot (bd + 2) + one look-ahead round + a window
    sess = _session(model, device, P + max_new_tokens + 3 * (bd + 2) + PAGE)
    eng = sess.eng
    dec = sess.decoder(bd, mask_id)
    if max_new_tokens <= 0:
        return [], dec, eos_id, device
    seed_logit = _prefill(eng, emb, positions)
    a0 = _argmax_rows(eng, seed_logit.view(1, -1), softmax_rule=True)
    dec.start(a0, pos_delta=torch.full((1,), next_pos - P, dtype=torch.int32, device=device))
    return _run_rounds(sess, dec, (bd, mask_id), bd, max_new_tokens, eos_id), dec, eos_id, device


def _finish(model, log_rows, dec, eos_id, device, bd, return_stats, trace, seed_key):
    """Committed ids, the trace entries and the text / stats of the drop-ins (src/fast_sampling.py:608-628)."""
    n_rounds = len(log_rows)
    committed: List[int] = []
    for row in log_rows:
        committed.append(row[0])
        committed.extend(row[2:3 + row[1]])
    if trace is not None:
        am = dec.log_am[:n_rounds, 0].cpu().tolist()
        tg = dec.log_tgt[:n_rounds, 0].cpu().tolist()
        for r, row in enumerate(log_rows):
            acc = row[1]
            k = bd + 1 if acc == bd else acc + 1
            ar_pred = [am[r][0]] + tg[r][:bd]
            entry = {"round": r + 1, "k": k}
            if seed_key:
                entry["seed"] = ar_pred[0]
            entry.update({"draft": am[r], "ar_pred": ar_pred, "new_tokens": [row[0]] + row[2:3 + acc]})
            trace.append(entry)
    gen = committed
    if eos_id is not None and eos_id in gen:
        gen = gen[:gen.index(eos_id)]
    txt = _decode_text(model, gen, device)
    if return_stats:
        fwd = 2 * n_rounds
        return txt, {"rounds": n_rounds, "draft_fwd": n_rounds, "verify_fwd": n_rounds, "commit_fwd": 0,
                     "total_fwd": fwd, "resp_tokens": len(gen), "tokens_per_fwd": round(len(gen) / max(1, fwd), 3),
                     "accept_per_round": round(len(committed) / max(1, n_rounds), 2)}
    return txt


@torch.no_grad()
def generate_speculative_natcache(model, image, prompt="Text Recognition:", max_new_tokens=512,
                                  draft_threshold=0.9, temperature=0.0, top_p=0.95,
                                  max_long_side=1344, accept_conf=0.0, draft_steps=1,
                                  return_stats=False, trace=None, draft_bd=None, full_draft=True):
    """O(N) cached self-speculative decode (src/fast_sampling.py:425-628) on the MI355X kernels.

    Same arguments, return value (text, or (text, stats) with the reference's stats keys) and ``trace`` entries
    ({"round", "k", "draft", "ar_pred", "new_tokens"} per round). ``draft_threshold`` and ``top_p`` are read only by
    the reference's iterative-unmask and sampling branches, which this path rejects (see the module docstring).
    """
    _check_greedy(temperature, accept_conf, draft_steps, full_draft)
    bd = int(draft_bd) if draft_bd else int(model.bd_size)
    rows, dec, eos_id, device = _spec_rounds(model, image, prompt, max_new_tokens, max_long_side, bd)
    return _finish(model, rows, dec, eos_id, device, bd, return_stats, trace, seed_key=False)


@torch.no_grad()
def generate_speculative_prefixcache(model, image, prompt="Text Recognition:", max_new_tokens=512,
                                     draft_threshold=0.9, temperature=0.0, top_p=0.95,
                                     max_long_side=1344, accept_conf=0.0, draft_steps=1,
                                     return_stats=False, trace=None, full_draft=True):
    """The prefix-cached self-speculative decode (src/fast_sampling.py:262-422) on the MI355X kernels: same
    arguments, return value and stats keys; ``trace`` entries {"round", "k", "seed", "draft", "ar_pred",
    "new_tokens"}.

    The reference caches only the prompt and re-forwards the committed response every round, the draft under a
    bd-grid block-causal mask and the verify causally (:325-338). Its committed ids are those of the causal
    verify, i.e. AR greedy decoding (:391-416); the draft's mask decides only how many of them a round accepts.
    Here the rounds are the engine's cached full-draft rounds (the committed response's K/V kept, not re-forwarded;
    the draft [pending | MASK x bd] against it), so the committed ids are the same AR greedy ids while the
    per-round acceptance, and with it ``rounds`` / ``accept_per_round`` and the trace's draft entries, follow the
    cached draft. Greedy, one draft step, full draft only, as the natcache drop-in."""
    _check_greedy(temperature, accept_conf, draft_steps, full_draft)
    bd = int(model.bd_size)
    rows, dec, eos_id, device = _spec_rounds(model, image, prompt, max_new_tokens, max_long_side, bd)
    return _finish(model, rows, dec, eos_id, device, bd, return_stats, trace, seed_key=True)


def _run_rounds(sess: _Session, dec: SelfSpecDecoder, key, bd: int, max_new_tokens: int, eos_id) -> List[List[int]]:
    """Round 0, then graph-replayed rounds until a round commits EOS or the committed count reaches the budget
    (the reference's loop condition, src/fast_sampling.py:499 and :614-616). Each round's packed row
    (a0, acc, t_0..t_acc) is copied to pinned memory behind the round; the host reads round r while round r + 1 runs
    whenever the budget alone cannot end at round r, so at most one round past an EOS is computed and discarded.
    Returns the packed rows of the rounds that count."""
    device = dec.eng.device
    stream = torch.cuda.current_stream(device)
    pin = [torch.empty(tuple(dec.st.packed.shape), dtype=torch.int32).pin_memory() for _ in range(2)]
    evs = [torch.cuda.Event() for _ in range(2)]
    issued = 0

    def issue():
        nonlocal issued
        if issued == 0:
            dec.round0()
        elif sess.graphed[key]:
            dec.g_round.replay()
        else:
            dec.round()                       # the first round runs eagerly, then it is captured for the rest
            torch.cuda.synchronize(device)
            _capture_round(dec)
            sess.graphed[key] = True
        pin[issued % 2].copy_(dec.st.packed, non_blocking=True)
        evs[issued % 2].record(stream)
        issued += 1

    rows: List[List[int]] = []
    n_committed = 0
    issue()
    while True:
        r = len(rows)
        if issued == r + 1 and n_committed + bd + 2 < max_new_tokens:
            issue()                           # round r + 1 is needed unless round r commits EOS
        evs[r % 2].synchronize()
        row = pin[r % 2][0].tolist()
        new = [row[0]] + row[2:3 + row[1]]
        rows.append(row)
        n_committed += len(new)
        if (eos_id is not None and eos_id in new) or n_committed >= max_new_tokens:
            break
        if issued == r + 1:
            issue()
    torch.cuda.synchronize(device)
    return rows


@torch.no_grad()
def generate_cached(model, image, prompt="Text Recognition:", max_new_tokens=512,
                    threshold=0.99, temperature=0.0, top_p=0.95, max_long_side=1344, commit_trace=None,
                    commit_causal=False, commit_detail=None):
    """KV-cached block-diffusion decode (src/fast_sampling.py:105-258) on the MI355X kernels: blocks of
    ``model.bd_size`` positions, threshold unmasking against the frozen cache, one commit forward per block.

    Same arguments and return value (the decoded text). ``commit_trace`` receives the number of positions each
    probe forward unmasked; ``commit_detail`` receives the reference's records (the seed of every block, then per
    probe forward the unmasked positions, ids and confidences and ``pred_all`` over the masked positions). Greedy
    only (``temperature == 0``; ``top_p`` is read by the sampling branch alone)."""
    _check_greedy(temperature)
    device = _model_device(model)
    bd, mask_id = int(model.bd_size), int(model.mask_id)
    eos_id = model.tokenizer.eos_token_id
    input_ids, emb, positions, next_pos = prepare_prompt(model, image, prompt, max_long_side, device)
    P = input_ids.shape[1]
    num_blocks = (max_new_tokens + bd - 1) // bd
    sess = _session(model, device, P + num_blocks * bd + PAGE)
    seed = int(_argmax_rows(sess.eng, _prefill(sess.eng, emb, positions).view(1, -1), softmax_rule=True)[0])
    dec = sess.diffusion_decoder(1, bd, mask_id, threshold, commit_causal)
    dec.start(torch.tensor([seed]), pos_delta=torch.tensor([next_pos - P]))
    generated: List[int] = []
    done = False
    for blk in range(num_blocks):
        if done or (eos_id is not None and seed == eos_id):
            break
        frozen = P + blk * bd
        if commit_detail is not None:
            commit_detail.append({"block": int(frozen // bd), "step": len(commit_detail), "pos": [int(frozen)],
                                  "in_block_pos": [0], "tok": [int(seed)], "conf": [1.0], "is_seed": True})
        on_step = None
        if commit_trace is not None or commit_detail is not None:
            def on_step(frozen=frozen):
                _record_step(dec, frozen, bd, mask_id, commit_trace, commit_detail)
        blocks, seeds, _ = dec.decode_block([seed], on_step)
        seed = seeds[0]
        for t in blocks[0]:
            if eos_id is not None and t == eos_id:
                done = True
                break
            generated.append(t)
    return _decode_text(model, generated, device)


def _record_step(dec: BlockDiffusionDecoder, frozen: int, bd: int, mask_id: int, commit_trace, commit_detail):
    """commit_trace / commit_detail entries of one probe step of row 0 (src/fast_sampling.py:217-238). A position
    counts as unmasked when it was masked before the step and holds another id after it."""
    before, after = dec.before[0].tolist(), dec.block[0].tolist()
    if commit_trace is not None:
        commit_trace.append(int(dec.n_unmasked[0]))
    if commit_detail is None:
        return
    idx = [i for i in range(bd) if before[i] == mask_id and after[i] != mask_id]
    if not idx:
        return
    x1, conf = dec.x1[0].tolist(), dec.conf[0].tolist()
    mp = [i for i in range(bd) if before[i] == mask_id]
    commit_detail.append({"pred_all": {"pos": mp, "tok": [int(x1[i]) for i in mp],
                                       "conf": [round(float(conf[i]), 4) for i in mp]},
                          "block": int(frozen // bd), "step": len(commit_detail),
                          "pos": [int(frozen + i) for i in idx], "in_block_pos": idx,
                          "tok": [int(x1[i]) for i in idx], "conf": [round(float(conf[i]), 4) for i in idx]})


def _capture_round(dec: SelfSpecDecoder):
    """Capture the decoder's round as a HIP graph. The capture records the round's kernels without running them
    (capture does not execute), so the decoder state is unchanged by it."""
    dec.g_round = torch.cuda.CUDAGraph()
    with torch.cuda.graph(dec.g_round):
        dec.round()


@torch.no_grad()
def teacher_force_argmax(model, image, prompt, gen_ids, max_long_side=1344):
    """One causal forward over prompt + gen_ids; the greedy id at every response position
    (src/fast_sampling.py:631-690): result[i] is the token the causal model places at response position i given
    gen_ids[:i]."""
    device = _model_device(model)
    input_ids, emb, positions, next_pos = prepare_prompt(model, image, prompt, max_long_side, device)
    P = input_ids.shape[1]
    g = torch.as_tensor(list(gen_ids), dtype=torch.long, device=device)
    L = int(g.shape[0])
    if L == 0:
        return []
    tm = model.text_model
    emb_all = torch.cat([emb, tm.embed_tokens(g[None])[0].to(emb.dtype)], 0)
    pos_gen = (torch.arange(L, device=device, dtype=torch.int32) + next_pos)[:, None].expand(L, 3)
    pos_all = torch.cat([positions, pos_gen], 0).contiguous()
    sess = _session(model, device, P + L + PAGE)
    logits = _prefill(sess.eng, emb_all, pos_all, logits_rows=(P - 1, P + L - 1))
    return _argmax_rows(sess.eng, logits).long().cpu().tolist()


def enable_fused_flex(dynamic=True):
    """The reference compiles flex attention once with dynamic shapes (src/fast_sampling.py:50-75). The MI355X path
    has no flex attention and no tracing compiler (every shape runs the same hand-written kernels), so there is
    nothing to configure; kept so callers of the reference run unchanged. Returns None."""
    return None
