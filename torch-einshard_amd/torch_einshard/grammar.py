"""Parser for einshard expressions.

A hand-written PEG-style recursive-descent parser accepting the language of the
reference's Parsley grammar (reference: src/torch_einshard/grammar.py:9-31):

    ws            = (' ' | '\\r' | '\\n' | '\\t')*
    id            = letterOrDigit+
    mesh_id       = letterOrDigit+ ('-' letterOrDigit+)*
    axis          = id ws '/' ws mesh_id        -> Axis(id, mesh_id)
                  | id                          -> Axis(id)
    ellipsis      = '...'
    group         = '(' (ws axis)+ ws ')'
    axes          = (ws (group | ellipsis | axis))+
    partial       = ws '//' ws ( '(' ws mesh_id (ws ',' ws mesh_id)* ws ')' | mesh_id )
    annotation    = ws '[' ws item (ws ',' ws item)* ws ']'
    item          = 'param' | 'grad' ws '=' ws value | 'init_sync' ws '=' ws value
    value         = letterOrDigit+ ('-' letterOrDigit+)* (':' letterOrDigit+)?
    input_tensor  = axes partial? annotation?
    output_tensor = axes partial?
    map           = input_tensor ws (',' input_tensor ws)? '->' output_tensor   <end of input>

``letterOrDigit`` is ``str.isalnum()`` or ``'_'``.  Every alternative backtracks
on failure, exactly like a PEG; the whole input must be consumed, so trailing
whitespace after the output spec is rejected.  Semantic errors raised while
building nodes (duplicate annotation items, two ellipses in one spec) propagate
as ``ValueError``.

``parse_sharding`` memoises parses (LRU, 2048 entries) and hands out a fresh copy
of the AST on every call so callers may mutate it (reference grammar.py:36-63);
any failure is re-raised as ``ValueError("Invalid einshard expression ...")``.
"""

from functools import lru_cache

from .sharding import Axes, Axis, AxisGroup, EllipsisAxis, TensorAnnotation, TensorSpec

__all__ = ["parse_sharding", "sharding", "ParseError", "Axes"]

_WS = " \r\n\t"


class ParseError(Exception):
    """Syntax error in an einshard expression; ``position`` is a character index."""

    def __init__(self, text: str, position: int, expected: str) -> None:
        self.text = text
        self.position = position
        self.expected = expected
        shown = text[position:position + 12] if position < len(text) else "<end of input>"
        super().__init__(f"expected {expected} at position {position} (found {shown!r})")


def _is_word_char(ch: str) -> bool:
    return ch.isalnum() or ch == "_"


class _Parser:
    def __init__(self, text: str) -> None:
        self.text = text
        self.pos = 0
        # furthest failure, reported when the whole parse fails
        self.fail_pos = 0
        self.fail_expected = "an axis"

    # -- primitives -------------------------------------------------------
    def _fail(self, expected: str):
        if self.pos >= self.fail_pos:
            self.fail_pos = self.pos
            self.fail_expected = expected
        return None

    def _peek(self, offset: int = 0) -> str:
        index = self.pos + offset
        return self.text[index] if index < len(self.text) else ""

    def ws(self) -> None:
        text, pos = self.text, self.pos
        while pos < len(text) and text[pos] in _WS:
            pos += 1
        self.pos = pos

    def literal(self, token: str) -> bool:
        if self.text.startswith(token, self.pos):
            self.pos += len(token)
            return True
        self._fail(repr(token))
        return False

    def word(self):
        text, start = self.text, self.pos
        end = start
        while end < len(text) and _is_word_char(text[end]):
            end += 1
        if end == start:
            return self._fail("a name")
        self.pos = end
        return text[start:end]

    def hyphenated(self):
        """``letterOrDigit+ ('-' letterOrDigit+)*``"""
        head = self.word()
        if head is None:
            return None
        pieces = [head]
        while self._peek() == "-" and _is_word_char(self._peek(1)):
            self.pos += 1
            pieces.append(self.word())
        return "-".join(pieces)

    # -- axes ---------------------------------------------------------------
    def axis(self):
        name = self.word()
        if name is None:
            return None
        after_name = self.pos
        self.ws()
        if self._peek() == "/":
            self.pos += 1
            self.ws()
            mesh = self.hyphenated()
            if mesh is not None:
                return Axis(name, mesh)
        self.pos = after_name
        return Axis(name)

    def group(self):
        start = self.pos
        if not self.literal("("):
            return None
        members = []
        while True:
            save = self.pos
            self.ws()
            member = self.axis()
            if member is None:
                self.pos = save
                break
            members.append(member)
        if not members:
            self.pos = start
            return None
        self.ws()
        if not self.literal(")"):
            self.pos = start
            return None
        return AxisGroup(members)

    def ellipsis(self):
        if self.literal("..."):
            return EllipsisAxis()
        return None

    def axes(self):
        items = []
        while True:
            save = self.pos
            self.ws()
            item = self.group()
            if item is None:
                item = self.ellipsis()
            if item is None:
                item = self.axis()
            if item is None:
                self.pos = save
                break
            items.append(item)
        return Axes(items) if items else None

    # -- partials and annotations ----------------------------------------
    def partial(self):
        start = self.pos
        self.ws()
        if not self.literal("//"):
            self.pos = start
            return None
        self.ws()
        many_start = self.pos
        if self.literal("("):
            self.ws()
            first = self.hyphenated()
            if first is not None:
                names = [first]
                while True:
                    save = self.pos
                    self.ws()
                    if not self.literal(","):
                        self.pos = save
                        break
                    self.ws()
                    name = self.hyphenated()
                    if name is None:
                        self.pos = save
                        break
                    names.append(name)
                self.ws()
                if self.literal(")"):
                    return names
            self.pos = many_start
        single = self.hyphenated()
        if single is None:
            self.pos = start
            return None
        return [single]

    def annotation_value(self):
        value = self.hyphenated()
        if value is None:
            return None
        if self._peek() == ":" and _is_word_char(self._peek(1)):
            self.pos += 1
            value += ":" + self.word()
        return value

    def annotation_item(self):
        start = self.pos
        if self.literal("param"):
            return ("param", True)
        for key in ("grad", "init_sync"):
            self.pos = start
            if self.literal(key):
                self.ws()
                if self.literal("="):
                    self.ws()
                    value = self.annotation_value()
                    if value is not None:
                        return (key, value)
        self.pos = start
        return self._fail("an annotation item")

    def annotation(self):
        start = self.pos
        self.ws()
        if not self.literal("["):
            self.pos = start
            return None
        self.ws()
        first = self.annotation_item()
        if first is None:
            self.pos = start
            return None
        items = [first]
        while True:
            save = self.pos
            self.ws()
            if not self.literal(","):
                self.pos = save
                break
            self.ws()
            item = self.annotation_item()
            if item is None:
                self.pos = save
                break
            items.append(item)
        self.ws()
        if not self.literal("]"):
            self.pos = start
            return None
        return TensorAnnotation.from_items(items)

    # -- tensors and the whole map -------------------------------------------
    def input_tensor(self):
        axes = self.axes()
        if axes is None:
            return None
        partials = self.partial()
        annotation = self.annotation()
        return TensorSpec(axes, partials or [], annotation)

    def output_tensor(self):
        axes = self.axes()
        if axes is None:
            return None
        partials = self.partial()
        return TensorSpec(axes, partials or [])

    def map(self):
        first = self.input_tensor()
        if first is None:
            raise self._error()
        self.ws()
        second = None
        save = self.pos
        if self.literal(","):
            second = self.input_tensor()
            if second is None:
                self.pos = save
            else:
                self.ws()
        if not self.literal("->"):
            raise self._error()
        out = self.output_tensor()
        if out is None:
            raise self._error()
        if self.pos != len(self.text):
            self._fail("end of input")
            raise self._error()
        return (first, second, out)

    def _error(self) -> ParseError:
        return ParseError(self.text, self.fail_pos, self.fail_expected)


class _Grammar:
    """``sharding(expression).map()`` — direct access to the parser, unwrapped errors."""

    def __init__(self, text: str) -> None:
        self._text = text

    def map(self):
        return _Parser(self._text).map()


def sharding(expression: str) -> _Grammar:
    return _Grammar(expression)


def parse_sharding(expression):
    """Parse ``expression`` into ``(input_spec, second_input_spec_or_None, output_spec)``."""
    try:
        return _copy_result(_parse_cached(expression))
    except Exception as error:  # noqa: BLE001 - every failure is reported the same way
        raise ValueError(f"Invalid einshard expression {expression!r}: {error}") from error


@lru_cache(maxsize=2048)
def _parse_cached(expression):
    return _Parser(expression).map()


def _copy_result(result):
    return tuple(None if spec is None else _copy_spec(spec) for spec in result)


def _copy_spec(spec: TensorSpec) -> TensorSpec:
    return TensorSpec(Axes(_copy_item(item) for item in spec.axes), spec.partials, spec.annotation)


def _copy_item(item):
    if isinstance(item, AxisGroup):
        return AxisGroup(_copy_item(member) for member in item.axes)
    if isinstance(item, EllipsisAxis):
        return EllipsisAxis()
    return Axis(item.name, item.shard_dim)
