"""Independent numpy writers of gpt.c's on-disk formats, used by the tests.

  checkpoint  model.py:246-283 (write_model / write_tensors): int32 header[256]
              (magic 20240415, block_size, vocab_size, n_layers, n_heads,
              n_embd, number of shape words, steps), the shape words
              (ndims, dims...) of every parameter, then the float32 data;
  tokenizer   tokenizer.py:12-40: int32 header[256] (magic 20240415,
              vocab_size, eot_token), then per piece a length byte and the
              bytes;
  tokens      data/common.py:35-48: raw int32 ids.
"""
import numpy as np

MAGIC = 20240415


def write_checkpoint(path, cfg, params, step):
    """cfg = (block_size, vocab_size, n_layers, n_heads, n_embd)."""
    block, V, L, H, C = cfg
    header = np.zeros(256, np.int32)
    header[:6] = [MAGIC, block, V, L, H, C]
    shapes = []
    for p in params:
        shapes += [p.ndim] + list(p.shape)
    header[6] = len(shapes)
    header[7] = step
    with open(path, "wb") as f:
        f.write(header.tobytes())
        f.write(np.array(shapes, np.int32).tobytes())
        for p in params:
            f.write(np.ascontiguousarray(p, np.float32).tobytes())


def read_checkpoint(path):
    """(header[:8] as ints, list of float32 arrays)."""
    raw = open(path, "rb").read()
    header = np.frombuffer(raw[:1024], np.int32)
    assert header[0] == MAGIC
    n_shape = int(header[6])
    shapes = np.frombuffer(raw[1024:1024 + 4 * n_shape], np.int32)
    off, i, params = 1024 + 4 * n_shape, 0, []
    while i < n_shape:
        nd = int(shapes[i])
        shp = tuple(int(d) for d in shapes[i + 1:i + 1 + nd])
        n = int(np.prod(shp))
        params.append(np.frombuffer(raw[off:off + 4 * n], np.float32).reshape(shp).copy())
        off += 4 * n
        i += nd + 1
    assert off == len(raw)
    return [int(h) for h in header[:8]], params


def write_tokenizer(path, pieces, eot):
    header = np.zeros(256, np.int32)
    header[:3] = [MAGIC, len(pieces), eot]
    with open(path, "wb") as f:
        f.write(header.tobytes())
        for b in pieces:
            f.write(bytes([len(b)]) + b)


def write_tokens(path, ids):
    np.asarray(ids, np.int32).tofile(path)
