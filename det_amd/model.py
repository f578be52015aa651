"""A det GGUF model on the GPU over det_model.h (ctypes): the reference's Model (crates/det/src/model.rs:164-548)
with greedy picking.

    python -m det_amd.model <det.gguf> <id> [<id> ...] [--new N] [--ctx C] [--batch B]
"""
import ctypes
import os
import sys

import numpy as np

from . import ffi

_bound = False


def _lib():
    global _bound
    L = ffi.lib()
    if not _bound:
        c, P = ctypes, ctypes.c_void_p
        for name, (res, args) in {'det_model_load': (P, [c.c_char_p, c.c_int, c.c_int]),
                                  'det_model_free': (None, [P]), 'det_model_last_error': (c.c_char_p, []),
                                  'det_model_vocab': (c.c_int, [P]), 'det_model_pos': (c.c_int, [P]),
                                  'det_model_reset': (None, [P]),
                                  'det_model_forward': (c.c_int, [P, P, c.c_int]),
                                  'det_model_prefill': (c.c_int, [P, P, c.c_int]),
                                  'det_model_logits': (c.c_int, [P, P]),
                                  'det_model_argmax': (c.c_int, [P]),
                                  'det_model_generate': (c.c_int, [P, P, c.c_int, c.c_int, P, c.c_int, P])}.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _bound = True
    return L


class ModelError(RuntimeError):
    pass


def _ids(ids):
    return np.ascontiguousarray(np.asarray(ids, dtype=np.int32))


class Model:
    def __init__(self, path, max_ctx, max_batch):
        L = _lib()
        self.h = L.det_model_load(os.fsencode(str(path)), int(max_ctx), int(max_batch))
        if not self.h:
            raise ModelError(L.det_model_last_error().decode())
        self.vocab = L.det_model_vocab(self.h)

    def _check(self, rc):
        if rc < 0:
            raise ModelError(_lib().det_model_last_error().decode())
        return rc

    @property
    def pos(self):
        return _lib().det_model_pos(self.h)

    def reset(self):
        _lib().det_model_reset(self.h)

    def forward(self, ids):
        a = _ids(ids)
        self._check(_lib().det_model_forward(self.h, a.ctypes.data, len(a)))

    def prefill(self, ids):
        a = _ids(ids)
        self._check(_lib().det_model_prefill(self.h, a.ctypes.data, len(a)))

    def logits(self):
        out = np.zeros(self.vocab, np.float32)
        self._check(_lib().det_model_logits(self.h, out.ctypes.data))
        return out

    def argmax(self):
        return self._check(_lib().det_model_argmax(self.h))

    def generate(self, prompt, n_new, stop=()):
        """Model::generate with greedy picking; an empty prompt continues from the last forward's logits."""
        p, s = _ids(prompt), _ids(list(stop))
        out = np.zeros(max(int(n_new), 1), np.int32)
        n = self._check(_lib().det_model_generate(self.h, p.ctypes.data if len(p) else None, len(p), int(n_new),
                                                  s.ctypes.data if len(s) else None, len(s), out.ctypes.data))
        return out[:n].tolist()

    def close(self):
        if self.h:
            _lib().det_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


def main(argv):
    args, ids, opts, i = argv, [], {'--new': 16, '--ctx': 4096, '--batch': 512}, 1
    if not args:
        print(__doc__)
        return 2
    while i < len(args):
        if args[i] in opts:
            opts[args[i]] = int(args[i + 1])
            i += 2
        else:
            ids.append(int(args[i]))
            i += 1
    m = Model(args[0], opts['--ctx'], opts['--batch'])
    print(' '.join(str(t) for t in m.generate(ids, opts['--new'])))
    return 0


if __name__ == '__main__':
    sys.exit(main(sys.argv[1:]))
