"""Grammar byte table of a real vocabulary (tokenizer.rs:108-117
token_bytes_table) over the C ABI: from a tokenizer.json document or from the
vocab embedded in a GGUF file (gguf_vocab.rs:75-171). Host only."""
import ctypes as C
import os
from typing import List, Optional

import numpy as np

from ._lib import lib


class TokenTableError(ValueError):
    pass


class HostTokenTable:
    """CSR token bytes: offsets[ntab + 1], data, valid[ntab] (0 = None), eos
    (eos_token_id, tokenizer.rs:52-57; None when the vocab has none)."""

    def __init__(self, h):
        try:
            n, nb, eos = C.c_uint32(), C.c_uint32(), C.c_int64()
            lib().zs_token_table_info(h, C.byref(n), C.byref(nb), C.byref(eos))
            self.ntab = n.value

            def arr(ptr, ctype, count):
                if count == 0:
                    return np.zeros(0, np.dtype(ctype))
                return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), (count,)).copy()

            self.offsets = arr(lib().zs_token_table_offsets(h), C.c_uint32, n.value + 1)
            self.data = arr(lib().zs_token_table_bytes(h), C.c_uint8, nb.value)
            self.valid = arr(lib().zs_token_table_valid(h), C.c_uint8, n.value)
            self.eos = None if eos.value < 0 else int(eos.value)
            to, tb = C.c_void_p(), C.c_void_p()
            lib().zs_token_table_text(h, C.byref(to), C.byref(tb))
            self.text_offsets = arr(to.value, C.c_uint32, n.value + 1)
            self.text = arr(tb.value, C.c_uint8, int(self.text_offsets[-1]))
        finally:
            lib().zs_token_table_destroy(h)

    def decode_text(self, i: int) -> str:
        """decode([i]) (special tokens skipped, lossy UTF-8), as shown in logprobs."""
        if i >= self.ntab:
            return ""
        return bytes(self.text[self.text_offsets[i]:self.text_offsets[i + 1]]).decode("utf-8")

    def tokens(self) -> List[Optional[bytes]]:
        return [bytes(self.data[self.offsets[i]:self.offsets[i + 1]]) if self.valid[i] else None
                for i in range(self.ntab)]

    @classmethod
    def from_tokenizer_json(cls, source: str):
        """`source`: a path to tokenizer.json or the JSON text itself."""
        text = open(source, "rb").read() if os.path.exists(source) else source.encode("utf-8")
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        if lib().zs_token_table_from_json(text, len(text), C.byref(h), err, 1024) != 0:
            raise TokenTableError(err.value.decode("utf-8", "replace"))
        return cls(h)

    @classmethod
    def from_gguf(cls, path: str):
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        if lib().zs_token_table_from_gguf(path.encode(), C.byref(h), err, 1024) != 0:
            raise TokenTableError(err.value.decode("utf-8", "replace"))
        return cls(h)
