"""A tokenizer stand-in for the tool protocol tests: special tokens at
chosen ids, expressions decoded as sums of small numbers, text encoded one
id per character (all ids inside the vocabulary)."""


class ToolTokenizer:
    NAMES = ("<|python_start|>", "<|python_end|>", "<|output_start|>", "<|output_end|>", "<|assistant_end|>")

    def __init__(self, V, python_start, python_end, output_start, output_end, assistant_end, bos):
        self.V = V
        self.ids = dict(zip(self.NAMES, (python_start, python_end, output_start, output_end, assistant_end)))
        self.bos = bos

    def encode_special(self, s):
        return self.ids[s]

    def get_bos_token_id(self):
        return self.bos

    def decode(self, ids):
        return "+".join(str(int(i) % 50) for i in ids)

    def encode(self, text):
        return [(7 * ord(c) + 3) % self.V for c in text]

    def __call__(self, text, prepend=None):
        return ([self.bos] if prepend is not None else []) + self.encode(text)
