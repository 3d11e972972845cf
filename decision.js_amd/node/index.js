"use strict";
/* decision.js on MI355X, Node host: `const { D1 } = require(".../decision.js_amd/node")`. */
const { D1, softmax } = require("./d1");
const { DecoderEngine, packForest, groupMax } = require("./engine");
const { loadWeights, fileFetch } = require("./format");
const questions = require("./questions");
const dj = require("./dj");

module.exports = { D1, DecoderEngine, packForest, groupMax, loadWeights, fileFetch, softmax, questions, dj };
