"""The data and scoring boundary on the CPU: the fixed token format (utils/prepare_data.py:19-70), the
training row order (run.py:688), the strict state-dict check (utils/eval.py:31), and the oracle's eager
scorer forward (utils/eval.py:43-46).

gpt_forward_eager rounds every op's result to bf16 explicitly in fp32 arithmetic. It is pinned here
against an independent formulation: the same forward written with bf16 tensors, where torch's own CPU
bf16 ops do the rounding (each op computes in fp32 and rounds its result, the dtype flow that eager bf16
autocast produces on the GPU: rms_norm of a bf16 tensor returns bf16, a 0-dim fp32 parameter times a bf16
tensor is bf16, and so on). Dropping or adding one rounding moves per-token losses by ~1e-2 with the head
scaled x30, far outside the bit-exact bar used here.
"""
import hashlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from noise_amd import prepare_data as pd
from noise_amd.eval import check_state_dict
from oracle import model as om

BF = torch.bfloat16


def test_token_hash_is_int32_le_bytes_whatever_the_container():
    rows = torch.arange(-3, 2 * pd.SEQ - 3, dtype=torch.int64).view(2, pd.SEQ) * 7919
    want = hashlib.sha256(rows.numpy().astype('<i4').tobytes()).hexdigest()
    assert pd.token_hash(rows) == want
    assert pd.token_hash(rows.to(torch.int32)) == want
    assert pd.token_hash(rows.numpy()) == want
    # a non-contiguous view hashes its logical row-major order
    assert pd.token_hash(rows.t().contiguous().t()) == want
    assert pd.token_hash(rows.flip(0)) != want


def test_load_rows_checks_shape_and_pinned_hash(tmp_path):
    good_shape = torch.zeros(pd.VAL_ROWS, pd.SEQ, dtype=torch.int32)
    torch.save(good_shape, tmp_path / 'val.pt')
    with pytest.raises(ValueError, match='hash mismatch'):
        pd.load_rows(tmp_path / 'val.pt', pd.VAL_ROWS)
    torch.save(torch.zeros(3, pd.SEQ, dtype=torch.int32), tmp_path / 'val.pt')
    with pytest.raises(ValueError, match='expected a'):
        pd.load_rows(tmp_path / 'val.pt', pd.VAL_ROWS)
    torch.save({'tokens': good_shape}, tmp_path / 'val.pt')
    with pytest.raises(ValueError, match='expected a'):
        pd.load_rows(tmp_path / 'val.pt', pd.VAL_ROWS)


def test_load_rows_accepts_the_pinned_tokens(tmp_path, monkeypatch):
    rows = torch.randint(0, 4096, (pd.VAL_ROWS, pd.SEQ), generator=torch.Generator().manual_seed(5),
                         dtype=torch.int32)
    monkeypatch.setitem(pd.EXPECTED, 'val.pt', pd.token_hash(rows))
    torch.save(rows, tmp_path / 'val.pt')
    got = pd.load_rows(tmp_path / 'val.pt', pd.VAL_ROWS)
    assert got.dtype == torch.int64 and torch.equal(got, rows.long())


def test_verify_reports_mismatch(tmp_path, capsys):
    torch.save(torch.zeros(pd.TRAIN_ROWS, pd.SEQ, dtype=torch.int32), tmp_path / 'train.pt')
    torch.save(torch.zeros(pd.VAL_ROWS, pd.SEQ, dtype=torch.int32), tmp_path / 'val.pt')
    with pytest.raises(SystemExit):
        pd.verify(tmp_path)
    out = capsys.readouterr().out
    assert out.count('MISMATCH') == 2


def test_split_sizes_are_the_reference_token_counts():
    # prepare_data.py:22-23: 9,994,240 training and 1,114,112 validation predictions
    assert pd.TRAIN_ROWS * (pd.SEQ - 1) == 9_994_240
    assert pd.VAL_ROWS * (pd.SEQ - 1) == 1_114_112


class _Tok:
    """A stand-in tokenizer: one id per character, <|endoftext|> = 0."""

    def token_to_id(self, s):
        assert s == '<|endoftext|>'
        return 0

    def encode(self, text):
        class E:
            ids = [ord(c) for c in text]
        return E()


def test_encode_split_joins_documents_and_cuts_whole_rows():
    docs = iter([{'text': 'ab' * 700}, {'text': 'c' * 1500}, {'text': 'd' * 5000}])
    out = pd.encode_split(docs, _Tok(), 2900)  # 2,902 tokens after two documents
    flat = [0] + [97, 98] * 700 + [0] + [99] * 1500
    assert out.dtype == torch.int32 and tuple(out.shape) == (1, pd.SEQ)
    assert out.view(-1).tolist() == flat[:pd.SEQ]


def test_training_order_is_seeded_randperm():
    got = pd.training_order(pd.TRAIN_ROWS)
    want = torch.randperm(pd.TRAIN_ROWS, generator=torch.Generator().manual_seed(1))
    assert torch.equal(got, want)
    assert torch.equal(got.sort().values, torch.arange(pd.TRAIN_ROWS))


def test_state_dict_check_names_what_differs():
    from noise_amd.model import GPT, GPTConfig
    with torch.device('meta'):
        sd = GPT(GPTConfig()).state_dict()
    check_state_dict(sd)
    bad = dict(sd)
    del bad['lm_head.weight']
    bad['extra.weight'] = torch.empty(1, device='meta')
    bad['transformer.h.0.attn.c_q.weight'] = torch.empty(512, 256, device='meta')
    with pytest.raises(RuntimeError) as e:
        check_state_dict(bad)
    msg = str(e.value)
    assert "missing keys ['lm_head.weight']" in msg
    assert "unexpected keys ['extra.weight']" in msg
    assert 'transformer.h.0.attn.c_q.weight: (512, 256) vs (512, 512)' in msg


def _dtype_driven_forward(P, idx, targets):
    """utils/model.py:193-209 written with bf16 tensors: torch's bf16 ops round each result."""
    B, T = idx.shape
    cos, sin = om.rotary_tables(T)
    c, s = cos.to(BF)[None, :, None, :], sin.to(BF)[None, :, None, :]
    W = {k: v.to(BF) for k, v in P.items()}
    lin = lambda x, n: (x.float() @ W[n].float().t()).to(BF)

    def rot(u):
        u1, u2 = u[..., :32], u[..., 32:]
        return torch.cat([u1 * c + u2 * s, u1 * -s + u2 * c], 3)

    x = x0 = F.rms_norm(W['transformer.wte.weight'][idx], (512,))
    for i in range(8):
        pre = f'transformer.h.{i}.'
        x = P['resid_lambdas'][i] * x + P['x0_lambdas'][i] * x0
        assert x.dtype == BF
        h = F.rms_norm(x, (512,))
        q, k, v = (lin(h, pre + f'attn.c_{n}.weight').view(B, T, 8, 64) for n in 'qkv')
        if om.has_ve(i):
            ve = W[f'value_embeds.{i}.weight'][idx].view(B, T, 8, 64)
            v = v + 2 * torch.sigmoid(lin(h[..., :32], pre + 'attn.ve_gate.weight')).unsqueeze(-1) * ve
        q, k = F.rms_norm(rot(q), (64,)), F.rms_norm(rot(k), (64,))
        y = om.attention(q.float(), k.float(), v.float(), om.window_sizes()[i]).to(BF).reshape(B, T, 512)
        x = x + lin(y, pre + 'attn.c_proj.weight')
        x = x + lin(F.relu(lin(F.rms_norm(x, (512,)), pre + 'mlp.c_fc.weight')).square(), pre + 'mlp.c_proj.weight')
    logits = lin(F.rms_norm(x, (512,)), 'lm_head.weight')[..., :4096].float()
    return om.softcap_ce(logits, targets, 'none')


def test_eager_oracle_matches_bf16_dtype_flow():
    from noise_amd.model import make_model
    torch.set_num_threads(min(8, torch.get_num_threads()))
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    rows = torch.randint(0, 4096, (2, 257), generator=torch.Generator().manual_seed(7))
    idx, tgt = rows[:, :-1], rows[:, 1:]
    want = _dtype_driven_forward(P, idx, tgt)
    got = om.gpt_forward_eager(P, idx, tgt, 'none').view_as(want)
    assert torch.equal(got, want)
    # the roundings matter at this scale: the fp32 forward is visibly elsewhere
    fp32 = om.gpt_forward(P, idx, tgt, 'none').view_as(want)
    assert (fp32 - want).abs().max().item() > 5e-3
