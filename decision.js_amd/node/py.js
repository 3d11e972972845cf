"use strict";
/* Python's json.dumps of a JSON value on the Node host: the legend text of a score level for the encoder kinds
 * (omni-prompt.ts:16 `criterion`, py.ts pyDumps). Integral numbers print as Python ints, others as Python's
 * float repr: the shortest round-trip digits, in fixed notation from 1e-4 up to 1e16, else d.ddde±XX. */

function pyFloat(x) {
  if (Number.isNaN(x)) return "NaN";
  if (!Number.isFinite(x)) return x > 0 ? "Infinity" : "-Infinity";
  if (Number.isInteger(x) && Math.abs(x) < 1e16) return String(x);
  const [m, e] = x.toExponential().split("e"); // shortest digits that round-trip
  const exp = Number(e);
  if (exp < -4 || exp >= 16) return `${m}e${exp < 0 ? "-" : "+"}${String(Math.abs(exp)).padStart(2, "0")}`;
  const sign = x < 0 ? "-" : "", digits = m.replace("-", "").replace(".", "");
  if (exp < 0) return `${sign}0.${"0".repeat(-exp - 1)}${digits}`;
  const whole = digits.slice(0, exp + 1).padEnd(exp + 1, "0"), frac = digits.slice(exp + 1);
  return `${sign}${whole}.${frac || "0"}`;
}

/** json.dumps(v, ensure_ascii=False) with Python's default separators. */
function pyDumps(v) {
  if (v === null || v === undefined) return "null";
  if (typeof v === "boolean") return v ? "true" : "false";
  if (typeof v === "number") return Number.isInteger(v) && Math.abs(v) < 1e16 ? String(v) : pyFloat(v);
  if (typeof v === "string") return JSON.stringify(v);
  if (Array.isArray(v)) return `[${v.map(pyDumps).join(", ")}]`;
  return `{${Object.entries(v).map(([k, x]) => `${JSON.stringify(k)}: ${pyDumps(x)}`).join(", ")}}`;
}

/** A score level's legend text for every kind but d1-3b: the text itself, else its json.dumps. */
const criterion = (v) => (typeof v === "string" ? v : pyDumps(v));

module.exports = { pyDumps, pyFloat, criterion };
