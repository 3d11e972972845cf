"use strict";
/* Questions and typed answers (questions.ts): {type: "noul" | "choice" | "score", instructions, criteria}.
 *   noul    yes/no; answer {noul: P(yes)}
 *   choice  one of >= 2 named options
 *   score   a level on a scale of 2 to 10 */

class QuestionError extends Error {}

/** Throws on a malformed question, as checkQuestion does (questions.ts:19-29). */
function checkQuestion(q) {
  if (!q || typeof q !== "object" || !("type" in q) || !("instructions" in q)) {
    throw new QuestionError("decision.js: a question is an object with `type`, `instructions` and, for choice and score, `criteria`");
  }
  const t = q.type, c = q.criteria;
  if (t !== "noul" && t !== "choice" && t !== "score") throw new QuestionError(`decision.js: question type must be noul, choice or score, got ${JSON.stringify(t)}`);
  if (t === "choice" && (!c || typeof c !== "object" || Array.isArray(c) || Object.keys(c).length < 2)) {
    throw new QuestionError("decision.js: a choice needs criteria {name: description} with at least two options");
  }
  if (t === "score" && (!Array.isArray(c) || c.length < 2 || c.length > 10)) {
    throw new QuestionError("decision.js: a score needs criteria: a list of 2 to 10 level descriptions, lowest first");
  }
  if (t === "noul" && c !== undefined && c !== null && (typeof c !== "object" || Array.isArray(c))) {
    throw new QuestionError('decision.js: noul criteria are optional: {"true": "...", "false": "..."} (or "yes", "no")');
  }
  return q;
}

const nOptions = (q) => (q.type === "noul" ? 2 : Array.isArray(q.criteria) ? q.criteria.length : Object.keys(q.criteria).length);

/** A question's typed answer from its probabilities ([yes, no] for a noul, else option order)
 * (questions.ts:32-45). */
function answer(q, probs, legend = String) {
  if (q.type === "noul") return { type: "noul", noul: probs[0] };
  let best = 0;
  probs.forEach((p, i) => {
    if (p > probs[best]) best = i;
  });
  if (q.type === "choice") {
    const names = Object.keys(q.criteria);
    const probabilities = {};
    names.forEach((n, i) => (probabilities[n] = probs[i]));
    return { type: "choice", choice: names[best], confidence: probs[best], probabilities };
  }
  const probabilities = {}, leg = {};
  probs.forEach((p, i) => (probabilities[String(i)] = p));
  q.criteria.forEach((c, i) => (leg[String(i)] = legend(c)));
  return { type: "score", score: probs.reduce((a, p, i) => a + i * p, 0), confidence: probs[best], probabilities, legend: leg };
}

module.exports = { QuestionError, checkQuestion, nOptions, answer };
