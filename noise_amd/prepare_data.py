"""The fixed token data format of utils/prepare_data.py, for reading and checking existing files.

  SEQ, TRAIN_ROWS, VAL_ROWS, EXPECTED      prepare_data.py:19-30 (row length, split sizes, pinned hashes)
  token_hash(rows)                         prepare_data.py:35-36
  load_rows(path, rows)                    prepare_data.py:39-47
  encode_split(documents, tokenizer, n)    prepare_data.py:50-57
  verify(out)                              prepare_data.py:60-70
  training_order(n, seed)                  train/val/run.py:688, eggroll.py:192 (the seeded shuffle)

A split is a [rows, 2049] integer tensor saved with torch.save: 2,048 predictions per row, token t's
target is token t + 1 of the same row. Its identity is the sha256 of the int32 little-endian token bytes,
independent of the container, so a file re-saved in another dtype or layout still verifies. Fetching and
tokenizing FineWeb (prepare_data.py:73-107) needs the network and is not reproduced here.
"""
import hashlib
from pathlib import Path

import numpy as np
import torch

SEQ = 2049
TRAIN_ROWS = 4880        # 9,994,240 prediction tokens
VAL_ROWS = 544           # 1,114,112 prediction tokens
SEED = 0                 # the training scripts' seed; the shuffle uses SEED + 1

EXPECTED = {
    'train.pt': '36ccb57eba6f5474b18acf99edd4a4793187260f7da7cc7053322cce59154bde',
    'val.pt': '5fdb9242ce8ab83e519ab5dd5cf8d64f4d8a99f6e74c137f4ca0f723da5f7437',
}


def token_hash(rows):
    """sha256 hex digest of the tokens as int32 little-endian, row-major."""
    data = rows.to(torch.int32).contiguous().numpy() if isinstance(rows, torch.Tensor) else np.asarray(rows)
    return hashlib.sha256(np.ascontiguousarray(data, dtype='<i4').tobytes()).hexdigest()


def load_rows(path, rows):
    """A fixed split as int64 [rows, 2049]. Raises ValueError for any other shape and, when the file name
    has a pinned hash, for other tokens. The file is read with torch.load(weights_only=True)."""
    data = torch.load(path, map_location='cpu', weights_only=True)
    if not isinstance(data, torch.Tensor) or tuple(data.shape) != (rows, SEQ):
        raise ValueError(f'{path}: expected a [{rows}, {SEQ}] token tensor')
    expected = EXPECTED[Path(path).name]
    if expected is not None and token_hash(data) != expected:
        raise ValueError(f'{path}: token hash mismatch; the file is not the pinned split')
    return data.long()


def encode_split(documents, tokenizer, min_tokens):
    """Documents joined by <|endoftext|> (one before each) until min_tokens, cut to whole rows:
    int32 [n, SEQ]. `documents` yields {'text': str}; `tokenizer` is a tokenizers.Tokenizer."""
    end = tokenizer.token_to_id('<|endoftext|>')
    tokens = []
    while len(tokens) < min_tokens:
        tokens.append(end)
        tokens.extend(tokenizer.encode(next(documents)['text']).ids)
    usable = len(tokens) // SEQ * SEQ
    return torch.tensor(tokens[:usable], dtype=torch.int32).view(-1, SEQ)


def verify(out):
    """Check out/train.pt and out/val.pt against their shapes and pinned hashes, printing one line each;
    SystemExit when either mismatches."""
    out = Path(out)
    ok = True
    for name, rows in (('train.pt', TRAIN_ROWS), ('val.pt', VAL_ROWS)):
        data = torch.load(out / name, map_location='cpu', weights_only=True)
        digest = token_hash(data)
        expected = EXPECTED[name]
        status = 'unpinned' if expected is None else ('OK' if digest == expected else 'MISMATCH')
        ok &= status != 'MISMATCH' and tuple(data.shape) == (rows, SEQ)
        print(f'{out / name}: {tuple(data.shape)} sha256 {digest} [{status}]', flush=True)
    if not ok:
        raise SystemExit('data does not match the pinned hashes')


def training_order(n, seed=SEED + 1):
    """The training scripts' row order: torch.randperm(n) on a CPU generator seeded with `seed`
    (run.py:688 / eggroll.py:192 draw it with SEED + 1 before the first step)."""
    return torch.randperm(n, generator=torch.Generator().manual_seed(seed))
