"""Hash-chained, append-only receipt log: the CIS-2 service's log format
(code/cis2-llm/server/app/receipts.py:31-97), for hosts that drive the
decode through the Python mirror.  The CLI writes and checks the same
format (cis2_host --receipt-log / --verify-chain).

Format: one JSON object per line.  prev_hash is the previous line's
log_hash (64 zeros for the first line); log_hash is the SHA-256 hex digest
of the record without log_hash, serialized with sorted keys, "," and ":"
separators and ASCII escapes.  Changing any field of a line breaks its
log_hash; removing or reordering lines breaks a prev_hash.
"""
import fcntl
import hashlib
import json
import os
import time
import uuid

GENESIS = "0" * 64


def canonical(record):
    """The bytes a record's log_hash covers."""
    return json.dumps(record, sort_keys=True, separators=(",", ":"), ensure_ascii=True).encode()


def _chain(lines, upto=None):
    """Checks JSON lines in order; returns (ok, message, head hash, records)."""
    prev, n = GENESIS, 0
    for text in lines:
        if not text.strip():
            continue
        try:
            rec = json.loads(text)
        except ValueError as e:
            return False, "line %d: not a JSON record (%s)" % (n, e), prev, n
        if not isinstance(rec, dict) or rec.get("prev_hash") != prev:
            return False, "line %d: prev_hash mismatch" % n, prev, n
        body = {k: v for k, v in rec.items() if k != "log_hash"}
        if rec.get("log_hash") != hashlib.sha256(canonical(body)).hexdigest():
            return False, "line %d: log_hash mismatch (tampered record)" % n, prev, n
        prev = rec["log_hash"]
        n += 1
        if upto is not None and rec.get("receipt_id") == upto:
            return True, "chain OK through line %d" % (n - 1), prev, n
    if upto is not None:
        return False, "receipt_id %s not found" % upto, prev, n
    return True, ("chain OK" if n else "empty log"), prev, n


class ReceiptLog:
    """A log file; appends hold an exclusive lock on it (several processes
    may append to one log) and refuse to extend a broken chain."""

    def __init__(self, path):
        self.path = os.fspath(path)

    def _lines(self):
        if not os.path.exists(self.path):
            return []
        with open(self.path, "r", encoding="utf-8") as f:
            return f.read().split("\n")

    def append(self, fields):
        """Appends a record with `fields` (plus prev_hash and log_hash) and
        returns it."""
        if "prev_hash" in fields or "log_hash" in fields:
            raise ValueError("prev_hash and log_hash are set by the log")
        with open(self.path, "a+", encoding="utf-8") as f:
            fcntl.flock(f, fcntl.LOCK_EX)
            try:
                f.seek(0)
                text = f.read()
                ok, msg, head, _ = _chain(text.split("\n"))
                if not ok:
                    raise RuntimeError("existing log is broken: " + msg)
                rec = dict(fields, prev_hash=head)
                rec["log_hash"] = hashlib.sha256(canonical(rec)).hexdigest()
                line = json.dumps(rec, sort_keys=True, ensure_ascii=True) + "\n"
                if text and not text.endswith("\n"):
                    line = "\n" + line
                f.write(line)
                f.flush()
                os.fsync(f.fileno())
            finally:
                fcntl.flock(f, fcntl.LOCK_UN)
        return rec

    def records(self):
        return [json.loads(t) for t in self._lines() if t.strip()]

    def get(self, receipt_id):
        for rec in self.records():
            if rec.get("receipt_id") == receipt_id:
                return rec
        return None

    def verify_chain(self, upto=None):
        """(ok, message) over the whole log, or through receipt `upto`."""
        ok, msg, _, _ = _chain(self._lines(), upto)
        return ok, msg


def decode_fields(model, result, prompt, reduction_mode=0, model_name=None):
    """The fields the CLI records for one decode (a Cis2Model.decode result):
    the witness and argmax digests, the table digests, the artifact hashes,
    the prompt and generated ids."""
    table, invf = (d.hex() for d in model.digests())
    hdr = model.hdr
    n = len(prompt)
    return {
        "receipt_id": uuid.uuid4().hex,
        "created": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
        "model": model_name or "cis2-%s-fp32" % model.spec.name,
        "cis2_version": "v0.4-candidate-tree" if reduction_mode else "v0.3b",
        "reduction_mode": "tree" if reduction_mode else "sequential",
        "backend": "gfx950",
        "witness_digest": result["witness"],
        "argmax_digest": result["argmax_digest"],
        "table_digest": table,
        "inv_freq_table_digest": invf,
        "weights_sha256": hdr[:32].hex(),
        "tokenizer_sha256": hdr[32:64].hex(),
        "config_sha256": hdr[64:96].hex(),
        "prompt_token_ids": [int(t) for t in prompt],
        "generated_token_ids": [int(t) for t in result["ids"][n:]],
    }
