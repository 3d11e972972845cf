"use strict";
/* decision.js on MI355X, Node host: `const { D1 } = require(".../decision.js_amd/node")` — the reference's
 * exports of index.ts: D1 (and its alias Decision), answer and checkQuestion, the engines. */
const { D1, Decision, softmax } = require("./d1");
const { DecoderEngine, packForest, packShared, groupMax } = require("./engine");
const { EncoderEngine, packEncoder } = require("./encoder");
const { OmniEngine, packOmni } = require("./omni");
const { LayaEngine, packLaya } = require("./laya");
const { D3Engine, gdnSpans } = require("./d3");
const { Eg2Engine } = require("./eg2");
const { Eg2Head } = require("./eg2_head");
const { loadWeights, fileFetch } = require("./format");
const questions = require("./questions");
const dj = require("./dj");

module.exports = {
  D1, Decision, answer: questions.answer, checkQuestion: questions.checkQuestion, DecoderEngine, EncoderEngine, OmniEngine,
  LayaEngine, D3Engine, Eg2Engine, Eg2Head, packForest, packShared, packEncoder, packOmni, packLaya, gdnSpans, groupMax, loadWeights, fileFetch, softmax, questions, dj,
};
