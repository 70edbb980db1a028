"""The sweep's text tables: one reader for every CSV this build consumes.

A table is a CSV file in which a line whose first character is '#' is not data.
Such a line is either provenance, written `# key,value` by ridge-measure (the
header and footer of a measured sweep), or free commentary. The first line that
is neither blank nor '#' is the header; every later line is a record with
exactly as many fields as the header names.

Registered shape lists (data/sweep/*-registered.csv, the format of the
reference's data/sweep/phase4-registered.csv) carry their header as a comment
and only `M,N,K,tag,rationale` records, so they have a reader of their own.

Errors are raised as TableError, which names the file and the 1-based line the
problem was found on, so that a malformed measurement is reported where it is,
not where a later computation trips over it.
"""

import csv
import re

_META_KEY = re.compile(r"^[A-Za-z_][A-Za-z0-9_]*$")


class TableError(ValueError):
    """A table that cannot be read as the caller needs it."""

    def __init__(self, path, line, problem):
        self.path, self.line, self.problem = path, line, problem
        where = "%s:%d" % (path, line) if line else str(path)
        super().__init__("%s: %s" % (where, problem))


class Table:
    """Header, records (dicts keyed by column name, values as written) and the
    `# key,value` provenance of one CSV file."""

    def __init__(self, path, columns, records, record_lines, meta):
        self.path = path
        self.columns = columns
        self.records = records
        self.record_lines = record_lines
        self.meta = meta

    def __len__(self):
        return len(self.records)

    def __iter__(self):
        return iter(self.records)

    def require(self, *names):
        """Raises TableError unless every named column is present."""
        absent = [n for n in names if n not in self.columns]
        if absent:
            raise TableError(self.path, 0, "no column %s (columns: %s)" % (
                ", ".join(repr(a) for a in absent), ",".join(self.columns)))
        return self

    def number(self, i, name, kind=float):
        """Field `name` of record i converted by `kind`; a field that does not
        convert is reported with its line."""
        raw = self.records[i][name]
        try:
            return kind(raw)
        except ValueError:
            raise TableError(self.path, self.record_lines[i], "column %r holds %r, not a %s"
                             % (name, raw, kind.__name__)) from None


def _provenance(text):
    body = text[1:].strip()
    key, sep, value = body.partition(",")
    key = key.strip()
    if sep and _META_KEY.match(key):
        return key, value.strip()
    return None


def read(path, require=()):
    """The Table in `path`. Raises TableError on a ragged record, a missing
    header or a required column that is absent."""
    with open(path, newline="") as f:
        return parse(f, path, require)


def parse(lines, source, require=()):
    """The Table held by an iterable of text lines; `source` names it in errors."""
    columns, records, numbers, meta = None, [], [], {}
    for lineno, text in enumerate(lines, start=1):
        if text.startswith("#"):
            kv = _provenance(text)
            if kv:
                meta[kv[0]] = kv[1]
            continue
        if not text.strip():
            continue
        fields = next(csv.reader([text]))
        if columns is None:
            columns = [c.strip() for c in fields]
            continue
        if len(fields) != len(columns):
            raise TableError(source, lineno, "%d fields where the header names %d" % (len(fields), len(columns)))
        records.append(dict(zip(columns, fields)))
        numbers.append(lineno)
    if columns is None:
        raise TableError(source, 0, "no header line")
    return Table(source, columns, records, numbers, meta).require(*require)


def write(path, columns, records, comments=()):
    """Writes `records` (dicts) under `columns`, after `comments` as '#' lines."""
    with open(path, "w", newline="") as f:
        for c in comments:
            f.write("# %s\n" % c)
        w = csv.DictWriter(f, fieldnames=columns, lineterminator="\n", extrasaction="ignore")
        w.writeheader()
        for r in records:
            w.writerow(r)


def read_shapes(path):
    """The registered shapes of a `M,N,K,tag,rationale` list, in file order, as
    (M, N, K, tag) tuples. Raises TableError on a record whose M, N or K is not
    a positive integer, and when the list is empty."""
    shapes = []
    with open(path, newline="") as f:
        for lineno, text in enumerate(f, start=1):
            if text.startswith("#") or not text.strip():
                continue
            fields = next(csv.reader([text]))
            try:
                mnk = tuple(int(x) for x in fields[:3])
            except ValueError:
                mnk = ()
            if len(mnk) != 3 or min(mnk) <= 0:
                raise TableError(path, lineno, "a registered shape starts with three positive integers M,N,K")
            tag = fields[3].strip() if len(fields) > 3 else "%dx%dx%d" % mnk
            shapes.append(mnk + (tag,))
    if not shapes:
        raise TableError(path, 0, "registers no shape")
    return shapes
