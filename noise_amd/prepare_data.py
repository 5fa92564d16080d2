"""The fixed token data format of utils/prepare_data.py, for reading and checking existing files.

  SEQ, TRAIN_ROWS, VAL_ROWS, EXPECTED      prepare_data.py:19-30 (row length, split sizes, pinned hashes)
  token_hash(rows)                         prepare_data.py:35-36
  load_rows(path, rows)                    prepare_data.py:39-47 (the call site eggroll.py:26 / eval.py imports)
  encode_split(documents, tokenizer, n)    prepare_data.py:50-57 (document packing rule)
  verify(out)                              prepare_data.py:60-70 (exit status on a mismatch)
  training_order(n, seed)                  train/val/run.py:688, eggroll.py:192 (the seeded shuffle)

A split is a [rows, 2049] integer tensor saved with torch.save: 2,048 predictions per row, token t's
target is token t + 1 of the same row. Its identity is the sha256 of the int32 little-endian token bytes,
independent of the container, so a file re-saved in another dtype or layout still verifies. Fetching and
tokenizing FineWeb (prepare_data.py:73-107) needs the network and is not reproduced here.

Every check goes through one function, `split_problems`, which lists what is wrong with a candidate
tensor (wrong type, wrong shape, hash differing from the pin); `load_rows` raises on the first problem
and `verify` reports all of them per file.
"""
import hashlib
from dataclasses import dataclass
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
# file name -> rows of the split stored under it
SPLIT_ROWS = {'train.pt': TRAIN_ROWS, 'val.pt': VAL_ROWS}
END_OF_TEXT = '<|endoftext|>'


def token_hash(rows):
    """sha256 hex digest of the tokens as int32 little-endian, row-major (any tensor, array or nested list)."""
    if isinstance(rows, torch.Tensor):
        rows = rows.detach().cpu().numpy()
    le32 = np.ascontiguousarray(np.asarray(rows), dtype='<i4')
    return hashlib.sha256(memoryview(le32).cast('B')).hexdigest()


def split_problems(data, rows, name=None):
    """What keeps `data` from being the split of `rows` rows stored as file `name`: a list of messages,
    empty when it is acceptable. The hash is only compared when the shape is right and `name` has a pin."""
    if not isinstance(data, torch.Tensor):
        return [f'expected a [{rows}, {SEQ}] token tensor, found {type(data).__name__}']
    if tuple(data.shape) != (rows, SEQ):
        return [f'expected a [{rows}, {SEQ}] token tensor, found shape {list(data.shape)}']
    pin = EXPECTED.get(name) if name is not None else None
    if pin is not None:
        digest = token_hash(data)
        if digest != pin:
            return [f'token hash mismatch: sha256 {digest}, pinned {pin}']
    return []


def _read(path):
    # weights_only: a token file is data; nothing in it may run on load
    return torch.load(Path(path), map_location='cpu', weights_only=True)


def load_rows(path, rows):
    """A fixed split as int64 [rows, 2049]. Raises ValueError when the file holds anything but a tensor of
    that shape or, for a file name with a pinned hash, other tokens."""
    path = Path(path)
    data = _read(path)
    problems = split_problems(data, rows, path.name)
    if problems:
        raise ValueError(f'{path}: {problems[0]}')
    return data.to(torch.int64)


def encode_split(documents, tokenizer, min_tokens):
    """Pack documents into rows: each document contributes <|endoftext|> followed by its token ids, in
    order, until at least `min_tokens` tokens are collected; the stream is then cut to whole rows of SEQ.
    Returns int32 [n, SEQ]. `documents` is an iterator of {'text': str}; `tokenizer` a tokenizers.Tokenizer
    (anything with token_to_id and encode(text).ids)."""
    end = tokenizer.token_to_id(END_OF_TEXT)
    pieces, total = [], 0
    while total < min_tokens:
        ids = tokenizer.encode(next(documents)['text']).ids
        piece = np.empty(len(ids) + 1, dtype=np.int32)
        piece[0] = end
        piece[1:] = ids
        pieces.append(piece)
        total += piece.size
    stream = np.concatenate(pieces) if pieces else np.empty(0, dtype=np.int32)
    whole = (stream.size // SEQ) * SEQ
    return torch.from_numpy(stream[:whole].copy()).view(-1, SEQ)


@dataclass
class SplitReport:
    path: Path
    shape: tuple
    digest: str
    problems: list

    @property
    def status(self):
        if self.problems:
            return 'MISMATCH'
        return 'pinned' if EXPECTED.get(self.path.name) else 'unpinned'


def verify(out):
    """Check every split file under `out` (train.pt, val.pt) against its shape and pinned hash. Prints one
    report line per file and raises SystemExit if any file fails; returns the reports otherwise."""
    out = Path(out)
    reports = []
    for name, rows in SPLIT_ROWS.items():
        data = _read(out / name)
        digest = token_hash(data) if isinstance(data, torch.Tensor) else '-'
        shape = tuple(data.shape) if isinstance(data, torch.Tensor) else ()
        reports.append(SplitReport(out / name, shape, digest, split_problems(data, rows, name)))
    for r in reports:
        detail = '; '.join(r.problems) if r.problems else f'sha256 {r.digest}'
        print(f'[{r.status}] {r.path} {list(r.shape)}: {detail}', flush=True)
    failed = [r.path.name for r in reports if r.problems]
    if failed:
        raise SystemExit(f'token files do not match their pins: {", ".join(failed)}')
    return reports


def training_order(n, seed=SEED + 1):
    """The training scripts' row order: torch.randperm(n) on a CPU generator seeded with `seed`
    (run.py:688 / eggroll.py:192 draw it with SEED + 1 before the first step)."""
    return torch.randperm(n, generator=torch.Generator().manual_seed(seed))
