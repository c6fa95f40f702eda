"""Measurement and search harness around the FFN (restates performance/ of the reference):
run.py drives cases x candidate configurations, tune.py searches, collect.py times and
profiles, analyze.py writes the report.  Results go to results/<run_id>/."""
